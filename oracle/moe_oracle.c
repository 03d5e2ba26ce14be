/*
 * CPU oracle for the sorted mixture-of-experts block — TEST INFRASTRUCTURE ONLY.
 * It is the checker for the HIP path and the timed CPU baseline; the product never
 * links it.  Each function cites the reference file:line it restates.
 *
 * Rounding model (the reference's MLX dtype flow): every MLX primitive returns a
 * bf16 tensor; matmul-like and reduction primitives accumulate in fp32 inside.
 *
 * Parity status of each function (how it is pinned; see the tests named):
 *   orc_f32_to_bf16      IEEE round-to-nearest-even; tests/test_oracle_math.py
 *                        (exhaustive-pattern comparison with numpy float64 rounding)
 *   orc_expf             |err| <= 2 ulp vs float64 exp over [-80, 88.7];
 *                        tests/test_oracle_math.py
 *   orc_router_logits    fp64 brute force on small shapes; tests/test_oracle_stages.py
 *   orc_route_topk       reference KAT routing_and_combination.rs:12-68 ({3/7,4/7});
 *                        argpartition KAT numeric_operations.rs:268-300; invariants
 *                        (k distinct ids, every unselected p <= every selected p,
 *                        ties at the boundary go to the higher index); brute force;
 *                        slice order = libstdc++ std::nth_element with MLX's (value, index)
 *                        comparator, called directly (orc_argpartition_bf16, argpartition.cc;
 *                        tests/test_oracle_argpartition.py)
 *   orc_sort_assignments reference KATs routing_and_combination.rs:109-182 and
 *                        hermetic/sparse_experts.rs:5-36; numpy stable argsort
 *   orc_invert_assignment_order  hermetic/sparse_experts.rs:5-36 (values and errors)
 *   orc_qmm / orc_gather_qmm     quantized_operations.rs:5-135 (4/8-bit [2080,4160]),
 *                        :137-172 (5-bit zeros), :255-306 (gather [6240,8320,2080,4160]);
 *                        fp64 dequantize+matmul brute force; LSB-first packing
 *                        checked against an independent numpy bit-stream packer
 *   orc_swiglu           compiled_swiglu.rs vectors vs float64 closed form
 *   orc_sorted_weighted_sum / orc_unsorted_weighted_sum
 *                        KAT [133,134,120,121] (sparse_experts.rs:86-173,
 *                        routing_and_combination.rs:184-226); [5,7] (sparse_experts.rs:34-64);
 *                        sorted == restored-unsorted
 *   orc_combine_shared   KAT [12,20] (routing_and_combination.rs:12-68)
 *   orc_moe_block_forward  composition of the above; fp64 brute force of the whole
 *                        block on a tiny layer (within bf16 rounding)
 *   orc_add_rms_norm     fp64 closed form (<= 1 bf16 ulp per rounding step), constant rows,
 *                        unit RMS of the unweighted output, eps dominance;
 *                        tests/test_oracle_decoder.py
 *   orc_decoder_ffn_forward  composition (residual add, RMS norm, block, residual add)
 *   orc_f32_to_f16 / orc_f16_to_f32  IEEE binary16 round to nearest even; tests/test_oracle_verify.py
 *                        (numpy float16 conversion over random, subnormal, overflow and tie patterns)
 *   orc_verification_quantized_linear  fp64 dequantize+matmul brute force on the reference's test
 *                        geometries (target_verification_quantized_linear.rs tests, 4/5-bit, bf16/f16);
 *                        4- and 5-bit code order checked against the reference QMV's byte masks
 *                        (target_verification_quantized_linear.rs:63-90); tests/test_oracle_verify.py
 *   orc_laguna_route     reference KATs laguna_hermetic/routing.rs:8-60 (bias selects only,
 *                        ties to the lower id, softcap before sigmoid, normalisation) and
 *                        direct_mlx/laguna/routing.rs:63-122 ([0, 1] with bias); fp64 brute force
 * Reference choices that only an MLX build could pin (MLX 0.32.1 is not vendored):
 * MLX's CPU exp/sum order inside softmax and its accumulation order in quantized matmul.
 * The in-slice order of argpartition is the C++ library's nth_element (called directly);
 * that MLX's CPU argpartition calls std::nth_element with the (value, index) comparator
 * is recalled from MLX's source, not pinned by a file here.  The choices made here are stated at each
 * function.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_LANES 64 /* canonical reduction width of the softmax denominator */

static int g_threads = 1;

void orc_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }
int orc_get_threads(void) { return g_threads; }

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float bf(uint16_t h) { return orc_bf16_to_f32(h); }
static inline uint16_t tobf(float f) { return orc_f32_to_bf16(f); }

/* IEEE binary16 from binary32, round to nearest even (subnormals, overflow to infinity). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds past 65504 */
  const int32_t e = (int32_t)(a >> 23) - 127;
  if (e >= -14) {
    const uint32_t m = a & 0x7fffffu, rest = m & 0x1fffu;
    uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
  }
  if (e < -25) return (uint16_t)sign;
  /* subnormal: value in units of 2^-24 is the 24-bit significand shifted right by -(e + 1) */
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const int32_t sh = -(e + 1);
  uint32_t h = m >> sh;
  const uint32_t rest = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (rest > half || (rest == half && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float f;
  if (e == 0) {
    f = ldexpf((float)m, -24);
    return sign ? -f : f;
  }
  const uint32_t u = sign | (e == 31 ? 0x7f800000u : (e + 112u) << 23) | (m << 13);
  memcpy(&f, &u, 4);
  return f;
}

/*
 * exp(x) for the softmax and sigmoid: Cody–Waite reduction x = n*ln2 + r with
 * |r| <= ln2/2, a degree-7 Taylor polynomial in Horner form (explicit fma), and an
 * exact power-of-two scale.  Results below e^-80 are flushed to 0 so no subnormal is
 * ever produced.  Every operation is an IEEE fp32 mul/fma/rint, so any IEEE
 * implementation of the same steps returns the same bits.
 */
float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283172607421875f) return INFINITY;
  if (x < -80.0f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860676533018704e-6f, r);
  float p = (float)(1.0 / 5040.0);
  p = fmaf(p, r, (float)(1.0 / 720.0));
  p = fmaf(p, r, (float)(1.0 / 120.0));
  p = fmaf(p, r, (float)(1.0 / 24.0));
  p = fmaf(p, r, (float)(1.0 / 6.0));
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) {
    p *= 2.0f;
    ni -= 1;
  }
  uint32_t sb = (uint32_t)(ni + 127) << 23;
  float scale;
  memcpy(&scale, &sb, 4);
  return p * scale;
}

static inline float sigmoidf_det(float v) { return 1.0f / (1.0f + orc_expf(-v)); }

/* Row 1 (forward.rs:59-91): logits = bf16(x · W_rᵀ), fp32 accumulation. */
void orc_router_logits(const uint16_t *x, const uint16_t *w, int32_t T, int32_t H,
                       int32_t E, uint16_t *logits) {
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
  for (int32_t t = 0; t < T; ++t) {
    for (int32_t e = 0; e < E; ++e) {
      const uint16_t *xr = x + (size_t)t * H;
      const uint16_t *wr = w + (size_t)e * H;
      float acc = 0.0f;
      for (int32_t h = 0; h < H; ++h) acc = fmaf(bf(xr[h]), bf(wr[h]), acc);
      logits[(size_t)t * E + e] = tobf(acc);
    }
  }
}

/*
 * Row 2 (routing.rs:16-48): p = softmax(logits) (precise: fp32 inside, bf16 out);
 * top-k by argpartition(p, kth = E-k) sliced to [E-k, E); scores = take(p);
 * optional renormalisation s / sum(s).
 *
 * Softmax: m = max; e_i = exp(l_i - m); S = sum e_i; p_i = bf16(e_i * (1/S)) (MLX's
 * CPU softmax multiplies by the reciprocal of the normaliser).  The order of the
 * sum is canonical: lane j of 64 sums i = j, j+64, ... in order, then the 64 lane
 * sums are combined by the butterfly lane[j] = lane[j] + lane[j ^ off] for
 * off = 1, 2, 4, 8, 16, 32 and S is lane 0.
 *
 * Selection: MLX's CPU argpartition runs std::nth_element over the index vector
 * 0..E-1 with the comparator (value, index), so the selected set is the k largest
 * (p, index) pairs — a tie at the boundary goes to the higher expert index — and the
 * order inside the slice [E-k, E) is the one libstdc++'s introselect leaves
 * (orc_argpartition_bf16, argpartition.cc, calls it).
 *
 * Renormalisation: sum in fp32 in slice order, rounded to bf16 (sum_axis output),
 * then bf16(s / sum) with IEEE division.
 */
int orc_route_topk(const uint16_t *logits, int32_t T, int32_t E, int32_t k,
                   int32_t normalize, uint32_t *indices, uint16_t *scores,
                   uint16_t *probabilities) {
  if (E <= 0 || k <= 0 || k > E || T < 0) return ORC_ERR_GEOMETRY;
  int err = ORC_OK;
#pragma omp parallel num_threads(g_threads)
  {
    float *ex = (float *)malloc(sizeof(float) * (size_t)E);
    uint16_t *pb = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)E);
    uint32_t *part = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)E);
    if (!ex || !pb || !part) {
#pragma omp atomic write
      err = ORC_ERR_GEOMETRY;
    } else {
#pragma omp for schedule(static)
      for (int32_t t = 0; t < T; ++t) {
        const uint16_t *l = logits + (size_t)t * E;
        float m = -INFINITY;
        for (int32_t i = 0; i < E; ++i) m = fmaxf(m, bf(l[i]));
        float lane[ORC_LANES];
        for (int j = 0; j < ORC_LANES; ++j) lane[j] = 0.0f;
        for (int32_t i = 0; i < E; ++i) {
          ex[i] = orc_expf(bf(l[i]) - m);
        }
        for (int j = 0; j < ORC_LANES; ++j)
          for (int32_t i = j; i < E; i += ORC_LANES) lane[j] = lane[j] + ex[i];
        for (int off = 1; off < ORC_LANES; off <<= 1) {
          float next[ORC_LANES];
          for (int j = 0; j < ORC_LANES; ++j) next[j] = lane[j] + lane[j ^ off];
          for (int j = 0; j < ORC_LANES; ++j) lane[j] = next[j];
        }
        const float rcp = 1.0f / lane[0];
        for (int32_t i = 0; i < E; ++i) {
          pb[i] = tobf(ex[i] * rcp);
          if (probabilities) probabilities[(size_t)t * E + i] = pb[i];
        }
        /* argpartition(p, E - k)[E - k:] */
        orc_argpartition_bf16(pb, E, E - k, part);
        for (int32_t j = 0; j < k; ++j) indices[(size_t)t * k + j] = part[E - k + j];
        uint16_t *s = scores + (size_t)t * k;
        const uint32_t *idx = indices + (size_t)t * k;
        for (int32_t j = 0; j < k; ++j) s[j] = pb[idx[j]];
        if (normalize) {
          float sum = 0.0f;
          for (int32_t j = 0; j < k; ++j) sum = sum + bf(s[j]);
          const float sb = bf(tobf(sum));
          for (int32_t j = 0; j < k; ++j) s[j] = tobf(bf(s[j]) / sb);
        }
      }
    }
    free(ex);
    free(pb);
    free(part);
  }
  return err;
}

/*
 * Row 3 (assignment_sort.rs:79-91): sorted_order = argsort(ids) with the index as
 * tie break (a stable sort), inverse_order = argsort(sorted_order),
 * sorted_ids = ids[sorted_order]; expert_offsets[e] = first sorted slot of expert e.
 */
int orc_sort_assignments(const uint32_t *ids, int32_t A, int32_t E,
                         uint32_t *sorted_order, uint32_t *inverse_order,
                         uint32_t *sorted_ids, uint32_t *expert_offsets) {
  if (A < 0 || E <= 0) return ORC_ERR_GEOMETRY;
  uint32_t *cursor = (uint32_t *)calloc((size_t)E + 1, sizeof(uint32_t));
  if (!cursor) return ORC_ERR_GEOMETRY;
  for (int32_t a = 0; a < A; ++a) {
    if (ids[a] >= (uint32_t)E) {
      free(cursor);
      return ORC_ERR_OUT_OF_RANGE;
    }
    cursor[ids[a] + 1]++;
  }
  for (int32_t e = 0; e < E; ++e) cursor[e + 1] += cursor[e];
  if (expert_offsets) memcpy(expert_offsets, cursor, sizeof(uint32_t) * ((size_t)E + 1));
  for (int32_t a = 0; a < A; ++a) {
    const uint32_t pos = cursor[ids[a]]++;
    if (sorted_order) sorted_order[pos] = (uint32_t)a;
    if (sorted_ids) sorted_ids[pos] = ids[a];
    if (inverse_order) inverse_order[a] = pos;
  }
  free(cursor);
  return ORC_OK;
}

/* Row 4 (assignment_permutation.rs:10-42). */
int orc_invert_assignment_order(const uint32_t *sorted_order, int32_t n,
                                uint32_t *inverse_order) {
  if (n < 0) return ORC_ERR_GEOMETRY;
  uint8_t *seen = (uint8_t *)calloc((size_t)n + 1, 1);
  if (!seen) return ORC_ERR_GEOMETRY;
  for (int32_t s = 0; s < n; ++s) {
    const uint32_t o = sorted_order[s];
    if (o >= (uint32_t)n) {
      free(seen);
      return ORC_ERR_OUT_OF_RANGE;
    }
    if (seen[o]) {
      free(seen);
      return ORC_ERR_DUPLICATE;
    }
    seen[o] = 1;
    inverse_order[o] = (uint32_t)s;
  }
  for (int32_t s = 0; s < n; ++s)
    if (!seen[s]) {
      free(seen);
      return ORC_ERR_MISSING;
    }
  free(seen);
  return ORC_OK;
}

static int affine_valid(const orc_affine *w) {
  if (!w || !w->w || !w->scales || !w->biases) return 0;
  if (w->bits != 2 && w->bits != 3 && w->bits != 4 && w->bits != 5 && w->bits != 6 &&
      w->bits != 8)
    return 0;
  if (w->group_size != 32 && w->group_size != 64 && w->group_size != 128) return 0;
  if (w->in_features <= 0 || w->out_features <= 0 || w->experts <= 0) return 0;
  if (w->in_features % w->group_size) return 0;
  if (((int64_t)w->in_features * w->bits) % 32) return 0;
  return 1;
}

/*
 * Row 5 packing (qwen3_5/artifacts/tensor_spec.rs:266-269, the QMV masks in
 * target_verification_quantized_linear.rs:28-35,63-70): element j of a row is bits
 * [j*b, j*b + b) of the row's little-endian bit stream of u32 words (LSB first).
 * Dequantised value: scale * q + bias per group of `group_size` inputs, in fp32.
 */
static void dequant_row_dt(const orc_affine *w, int32_t expert, int32_t n, float *out, int f16);

static void dequant_row_f32(const orc_affine *w, int32_t expert, int32_t n, float *out) {
  dequant_row_dt(w, expert, n, out, 0);
}

/* scales and biases read as bf16 (f16 == 0) or IEEE binary16 */
static void dequant_row_dt(const orc_affine *w, int32_t expert, int32_t n, float *out, int f16) {
  const int32_t K = w->in_features;
  const int32_t words = (int32_t)(((int64_t)K * w->bits) / 32);
  const int32_t groups = K / w->group_size;
  const uint32_t *row = w->w + ((size_t)expert * w->out_features + n) * (size_t)words;
  const uint16_t *sc = w->scales + ((size_t)expert * w->out_features + n) * (size_t)groups;
  const uint16_t *bi = w->biases + ((size_t)expert * w->out_features + n) * (size_t)groups;
  const uint32_t mask = (1u << w->bits) - 1u;
  for (int32_t j = 0; j < K; ++j) {
    const uint64_t bit = (uint64_t)j * (uint64_t)w->bits;
    const uint64_t word = bit >> 5;
    const uint32_t shift = (uint32_t)(bit & 31u);
    uint64_t v = row[word];
    if (shift + (uint32_t)w->bits > 32u) v |= (uint64_t)row[word + 1] << 32;
    const uint32_t q = (uint32_t)(v >> shift) & mask;
    const int32_t g = j / w->group_size;
    out[j] = f16 ? fmaf(orc_f16_to_f32(sc[g]), (float)q, orc_f16_to_f32(bi[g]))
                 : fmaf(bf(sc[g]), (float)q, bf(bi[g]));
  }
}

int orc_dequantize(const orc_affine *w, int32_t expert, uint16_t *out_bf16) {
  if (!affine_valid(w) || expert < 0 || expert >= w->experts) return ORC_ERR_GEOMETRY;
  float *row = (float *)malloc(sizeof(float) * (size_t)w->in_features);
  if (!row) return ORC_ERR_GEOMETRY;
  for (int32_t n = 0; n < w->out_features; ++n) {
    dequant_row_f32(w, expert, n, row);
    for (int32_t j = 0; j < w->in_features; ++j)
      out_bf16[(size_t)n * w->in_features + j] = tobf(row[j]);
  }
  free(row);
  return ORC_OK;
}

/* fp32 dot product with 8 interleaved fma accumulators, combined as a fixed tree. */
static inline float dot_f32(const float *a, const float *b, int32_t K) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int32_t j = 0;
  for (; j + 8 <= K; j += 8)
    for (int u = 0; u < 8; ++u) acc[u] = fmaf(a[j + u], b[j + u], acc[u]);
  for (; j < K; ++j) acc[0] = fmaf(a[j], b[j], acc[0]);
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

/*
 * Rows 5/8/11 (mlx_quantized_operations.rs:49-157, transpose = true):
 * y[m][n] = bf16( sum_j x[m][j] * deq(W[expert])[n][j] ) with fp32 accumulation.
 * `rows` lists the M activation rows that use `expert`; their outputs go to the same
 * row positions of y.  One dequantised weight row is shared by all listed rows.
 */
static void qmm_rows(const uint16_t *x, const int32_t *rows, int32_t nrows,
                     const orc_affine *w, int32_t expert, uint16_t *y) {
  const int32_t K = w->in_features, N = w->out_features;
  float *xf = (float *)malloc(sizeof(float) * (size_t)nrows * K);
  if (!xf) return;
  for (int32_t r = 0; r < nrows; ++r)
    for (int32_t j = 0; j < K; ++j) xf[(size_t)r * K + j] = bf(x[(size_t)rows[r] * K + j]);
#pragma omp parallel num_threads(g_threads)
  {
    float *wr = (float *)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int32_t n = 0; n < N; ++n) {
      dequant_row_f32(w, expert, n, wr);
      for (int32_t r = 0; r < nrows; ++r)
        y[(size_t)rows[r] * N + n] = tobf(dot_f32(xf + (size_t)r * K, wr, K));
    }
    free(wr);
  }
  free(xf);
}

int orc_qmm(const uint16_t *x, int32_t M, const orc_affine *w, int32_t expert,
            uint16_t *y) {
  if (!affine_valid(w) || M < 0 || expert < 0 || expert >= w->experts) return ORC_ERR_GEOMETRY;
  if (M == 0) return ORC_OK;
  int32_t *rows = (int32_t *)malloc(sizeof(int32_t) * (size_t)M);
  if (!rows) return ORC_ERR_GEOMETRY;
  for (int32_t m = 0; m < M; ++m) rows[m] = m;
  qmm_rows(x, rows, M, w, expert, y);
  free(rows);
  return ORC_OK;
}

/*
 * gather_qmm (gathered_projection.rs:84-131 -> mlx_gather_qmm with rhs indices):
 * y[r] = x[x_rows ? x_rows[r] : r] · deq(W[ids[r]])ᵀ.  Output row r keeps the caller's
 * order whether or not ids are sorted (the sorted flag only changes kernel choice).
 */
int orc_gather_qmm(const uint16_t *x, const uint32_t *x_rows, int32_t rows,
                   const orc_affine *w, const uint32_t *ids, uint16_t *y) {
  if (!affine_valid(w) || rows < 0) return ORC_ERR_GEOMETRY;
  const int32_t K = w->in_features, N = w->out_features;
  for (int32_t r = 0; r < rows; ++r)
    if (ids[r] >= (uint32_t)w->experts) return ORC_ERR_OUT_OF_RANGE;
  uint16_t *xs = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)rows * K + 1));
  uint16_t *ys = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)rows * N + 1));
  int32_t *list = (int32_t *)malloc(sizeof(int32_t) * ((size_t)rows + 1));
  if (!xs || !ys || !list) {
    free(xs); free(ys); free(list);
    return ORC_ERR_GEOMETRY;
  }
  for (int32_t r = 0; r < rows; ++r)
    memcpy(xs + (size_t)r * K, x + (size_t)(x_rows ? x_rows[r] : (uint32_t)r) * K,
           sizeof(uint16_t) * (size_t)K);
  for (int32_t e = 0; e < w->experts; ++e) {
    int32_t n = 0;
    for (int32_t r = 0; r < rows; ++r)
      if (ids[r] == (uint32_t)e) list[n++] = r;
    if (n) qmm_rows(xs, list, n, w, e, ys);
  }
  memcpy(y, ys, sizeof(uint16_t) * (size_t)rows * N);
  free(xs); free(ys); free(list);
  return ORC_OK;
}

/*
 * qwen3_5_target_verification_quantized_linear (qwen3_5/model/target_verification_quantized_linear.rs:
 * 232-330) over rows = batch * tokens activation rows, with the geometry checks of
 * validate_target_verification_projection (:378-447).  Every row is projected alone, as the
 * reference's token-local path does (:333-356): y[r][n] = round(sum_j x[r][j] * (s q + b)) with
 * fp32 accumulation and one rounding to the activations' dtype (bf16, or binary16 when f16).
 */
int orc_verification_quantized_linear(const uint16_t *x, int32_t rows, const orc_affine *w, int32_t f16,
                                      uint16_t *y) {
  if (!affine_valid(w) || w->experts != 1 || rows <= 0) return ORC_ERR_GEOMETRY;
  const int32_t K = w->in_features, N = w->out_features;
#pragma omp parallel num_threads(g_threads)
  {
    float *wr = (float *)malloc(sizeof(float) * (size_t)K);
    float *xr = (float *)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int32_t n = 0; n < N; ++n) {
      dequant_row_dt(w, 0, n, wr, f16);
      for (int32_t r = 0; r < rows; ++r) {
        for (int32_t j = 0; j < K; ++j) {
          const uint16_t h = x[(size_t)r * K + j];
          xr[j] = f16 ? orc_f16_to_f32(h) : bf(h);
        }
        const float v = dot_f32(xr, wr, K);
        y[(size_t)r * N + n] = f16 ? orc_f32_to_f16(v) : tobf(v);
      }
    }
    free(wr);
    free(xr);
  }
  return ORC_OK;
}

/* Row 7 (mlx_compiled_swiglu.rs:44-89): sigmoid, multiply, multiply — each bf16. */
void orc_swiglu(const uint16_t *gate, const uint16_t *up, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i) {
    const float g = bf(gate[i]);
    const float s = bf(tobf(sigmoidf_det(g)));
    const float a = bf(tobf(g * s));
    out[i] = tobf(a * bf(up[i]));
  }
}

/* Row 9 (weighted_sum.rs:16-33): fp32 sum over j in slot order of out·score, one
 * bf16 rounding at the end. */
void orc_sorted_weighted_sum(const uint16_t *sorted_out, const uint32_t *inverse_order,
                             const uint16_t *scores, int32_t T, int32_t k, int32_t D,
                             uint16_t *y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int32_t t = 0; t < T; ++t) {
    for (int32_t d = 0; d < D; ++d) {
      float acc = 0.0f;
      for (int32_t j = 0; j < k; ++j) {
        const size_t a = (size_t)t * k + j;
        acc = fmaf(bf(sorted_out[(size_t)inverse_order[a] * D + d]), bf(scores[a]), acc);
      }
      y[(size_t)t * D + d] = tobf(acc);
    }
  }
}

/* Row 10 (weighted_sum.rs:94-120): bf16 product out·score (multiply primitive), then
 * sum over the expert axis with fp32 accumulation in slot order, one bf16 rounding. */
void orc_unsorted_weighted_sum(const uint16_t *out, const uint16_t *scores, int32_t T,
                               int32_t k, int32_t D, uint16_t *y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int32_t t = 0; t < T; ++t) {
    for (int32_t d = 0; d < D; ++d) {
      float acc = 0.0f;
      for (int32_t j = 0; j < k; ++j) {
        const size_t a = (size_t)t * k + j;
        acc = acc + bf(tobf(bf(out[a * D + d]) * bf(scores[a])));
      }
      y[(size_t)t * D + d] = tobf(acc);
    }
  }
}

/* Row 12 (output_combination.rs:34-43): sparse + shared * sigmoid(gate), each bf16. */
void orc_combine_shared(const uint16_t *sparse, const uint16_t *shared_out,
                        const uint16_t *gate_logits, int32_t T, int32_t D, uint16_t *y) {
  for (int32_t t = 0; t < T; ++t) {
    const float g = bf(tobf(sigmoidf_det(bf(gate_logits[t]))));
    for (int32_t d = 0; d < D; ++d) {
      const size_t i = (size_t)t * D + d;
      const float gated = bf(tobf(bf(shared_out[i]) * g));
      y[i] = tobf(bf(sparse[i]) + gated);
    }
  }
}

#define MINIMUM_SORTED_EXPERT_ASSIGNMENTS 64 /* routing.rs:13 */

/* fused [E][2I] rows or separate gate/up: returns gate and up of the assignment rows */
static int expert_gate_up(const orc_layer *L, const uint16_t *x, const uint32_t *x_rows,
                          int32_t A, const uint32_t *ids, uint16_t *gate, uint16_t *up) {
  const int32_t I = L->intermediate;
  if (L->gate_up.w) {
    uint16_t *gu = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)A * 2 * I + 1));
    if (!gu) return ORC_ERR_GEOMETRY;
    int rc = orc_gather_qmm(x, x_rows, A, &L->gate_up, ids, gu);
    for (int32_t a = 0; a < A && rc == ORC_OK; ++a) {
      memcpy(gate + (size_t)a * I, gu + (size_t)a * 2 * I, sizeof(uint16_t) * (size_t)I);
      memcpy(up + (size_t)a * I, gu + (size_t)a * 2 * I + I, sizeof(uint16_t) * (size_t)I);
    }
    free(gu);
    return rc;
  }
  int rc = orc_gather_qmm(x, x_rows, A, &L->up, ids, up);
  if (rc == ORC_OK) rc = orc_gather_qmm(x, x_rows, A, &L->gate, ids, gate);
  return rc;
}

/*
 * Rows 1-13: Qwen3_5Model::forward_qwen3_5_moe (forward.rs:19-127) with the resident
 * owner (resident_execution.rs:70-143, :210-258, :352-400).
 */
int orc_moe_block_forward(const orc_layer *L, const uint16_t *x, int32_t T,
                          const uint16_t *logits_override, uint16_t *y,
                          orc_trace *trace) {
  const int32_t H = L->hidden, E = L->num_experts, k = L->top_k, I = L->intermediate;
  if (T < 0 || H <= 0 || E <= 0 || k <= 0 || k > E || I <= 0) return ORC_ERR_GEOMETRY;
  const int32_t A = T * k;
  int rc = ORC_OK;
  uint16_t *logits = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)T * E + 1));
  uint32_t *idx = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)A + 1));
  uint16_t *scores = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)A + 1));
  uint16_t *gate = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)A * I + 1));
  uint16_t *up = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)A * I + 1));
  uint16_t *act = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)A * I + 1));
  uint16_t *eout = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)A * H + 1));
  uint16_t *sparse = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)T * H + 1));
  uint32_t *sorted_order = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)A + 1));
  uint32_t *inverse = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)A + 1));
  uint32_t *sorted_ids = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)A + 1));
  uint32_t *x_rows = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)A + 1));
  uint32_t *offsets = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)E + 1));
  if (!logits || !idx || !scores || !gate || !up || !act || !eout || !sparse ||
      !sorted_order || !inverse || !sorted_ids || !x_rows || !offsets) {
    rc = ORC_ERR_GEOMETRY;
    goto done;
  }

  /* router projection, then the harness-only logit bias */
  if (logits_override) {
    memcpy(logits, logits_override, sizeof(uint16_t) * (size_t)T * E);
  } else {
    if (L->router_w) {
      orc_router_logits(x, L->router_w, T, H, E, logits);
    } else {
      rc = orc_qmm(x, T, &L->router_q, 0, logits);
      if (rc) goto done;
    }
    if (L->router_bias)
      for (int32_t t = 0; t < T; ++t)
        for (int32_t e = 0; e < E; ++e) {
          const size_t i = (size_t)t * E + e;
          logits[i] = tobf(bf(logits[i]) + bf(L->router_bias[e]));
        }
  }
  if (trace && trace->logits) memcpy(trace->logits, logits, sizeof(uint16_t) * (size_t)T * E);
  rc = orc_route_topk(logits, T, E, k, L->normalize_top_k, idx, scores,
                      trace ? trace->probabilities : NULL);
  if (rc) goto done;
  if (trace && trace->indices) memcpy(trace->indices, idx, sizeof(uint32_t) * (size_t)A);
  if (trace && trace->scores) memcpy(trace->scores, scores, sizeof(uint16_t) * (size_t)A);

  const int sorted = A >= MINIMUM_SORTED_EXPERT_ASSIGNMENTS;
  if (trace) trace->used_sorted_path = sorted;
  if (sorted) {
    /* assignment_sort.rs:79-91; sorted_states = x[sorted_order // k] */
    rc = orc_sort_assignments(idx, A, E, sorted_order, inverse, sorted_ids, offsets);
    if (rc) goto done;
    for (int32_t s = 0; s < A; ++s) x_rows[s] = sorted_order[s] / (uint32_t)k;
    rc = expert_gate_up(L, x, x_rows, A, sorted_ids, gate, up);
    if (rc) goto done;
    orc_swiglu(gate, up, (int64_t)A * I, act);
    rc = orc_gather_qmm(act, NULL, A, &L->down, sorted_ids, eout);
    if (rc) goto done;
    orc_sorted_weighted_sum(eout, inverse, scores, T, k, H, sparse);
    if (trace) {
      if (trace->sorted_order) memcpy(trace->sorted_order, sorted_order, sizeof(uint32_t) * (size_t)A);
      if (trace->inverse_order) memcpy(trace->inverse_order, inverse, sizeof(uint32_t) * (size_t)A);
      if (trace->sorted_ids) memcpy(trace->sorted_ids, sorted_ids, sizeof(uint32_t) * (size_t)A);
      if (trace->expert_offsets) memcpy(trace->expert_offsets, offsets, sizeof(uint32_t) * ((size_t)E + 1));
      for (int32_t a = 0; a < A; ++a) {
        if (trace->activated)
          memcpy(trace->activated + (size_t)a * I, act + (size_t)inverse[a] * I, sizeof(uint16_t) * (size_t)I);
        if (trace->expert_out)
          memcpy(trace->expert_out + (size_t)a * H, eout + (size_t)inverse[a] * H, sizeof(uint16_t) * (size_t)H);
      }
    }
  } else {
    /* unsorted: expanded states [1,T,1,1,H] broadcast over the k assignments */
    for (int32_t a = 0; a < A; ++a) x_rows[a] = (uint32_t)(a / k);
    rc = expert_gate_up(L, x, x_rows, A, idx, gate, up);
    if (rc) goto done;
    orc_swiglu(gate, up, (int64_t)A * I, act);
    rc = orc_gather_qmm(act, NULL, A, &L->down, idx, eout);
    if (rc) goto done;
    orc_unsorted_weighted_sum(eout, scores, T, k, H, sparse);
    if (trace) {
      if (trace->activated) memcpy(trace->activated, act, sizeof(uint16_t) * (size_t)A * I);
      if (trace->expert_out) memcpy(trace->expert_out, eout, sizeof(uint16_t) * (size_t)A * H);
    }
  }
  if (trace && trace->sparse) memcpy(trace->sparse, sparse, sizeof(uint16_t) * (size_t)T * H);

  if (L->shared_intermediate > 0) {
    const int32_t Is = L->shared_intermediate;
    uint16_t *sg = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)T * Is + 1));
    uint16_t *su = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)T * Is + 1));
    uint16_t *sa = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)T * Is + 1));
    uint16_t *so = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)T * H + 1));
    uint16_t *z = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)T + 1));
    if (!sg || !su || !sa || !so || !z) rc = ORC_ERR_GEOMETRY;
    if (!rc) rc = orc_qmm(x, T, &L->shared_gate, 0, sg);
    if (!rc) rc = orc_qmm(x, T, &L->shared_up, 0, su);
    if (!rc) orc_swiglu(sg, su, (int64_t)T * Is, sa);
    if (!rc) rc = orc_qmm(sa, T, &L->shared_down, 0, so);
    if (!rc) rc = orc_qmm(x, T, &L->shared_expert_gate, 0, z);
    if (!rc) orc_combine_shared(sparse, so, z, T, H, y);
    if (!rc && trace) {
      if (trace->shared_out) memcpy(trace->shared_out, so, sizeof(uint16_t) * (size_t)T * H);
      if (trace->shared_gate_logits) memcpy(trace->shared_gate_logits, z, sizeof(uint16_t) * (size_t)T);
    }
    free(sg); free(su); free(sa); free(so); free(z);
  } else {
    memcpy(y, sparse, sizeof(uint16_t) * (size_t)T * H);
  }

done:
  free(logits); free(idx); free(scores); free(gate); free(up); free(act); free(eout);
  free(sparse); free(sorted_order); free(inverse); free(sorted_ids); free(x_rows);
  free(offsets);
  return rc;
}

/*
 * The decoder step around the block (decoder_layer_forward.rs:111-174; the RMS norm of
 * mlx_fast_rms_norm, mlx_operations.rs:91-101): r = bf16(h + a) (a may be NULL: r = h);
 * n = bf16(w * bf16(r * inv)), inv = 1 / sqrt(mean(r^2) + eps) in fp32, IEEE sqrt and
 * division.  MLX computes the normaliser in fp32, rounds x * inv to the input dtype and
 * multiplies by the weight in that dtype (its fast::rms_norm fallback); the order of the
 * fp32 sum of squares inside MLX is not pinned.  This restatement fixes it: partial j of 256
 * owns the 8-element chunks j, j + 256, ... and sums their r_i^2 in element order; the
 * partials of each group of 64 combine by the butterfly of the softmax denominator, and the
 * four group sums as (g0 + g1) + (g2 + g3).  H is a multiple of 8.
 */
static void rms_norm_row(const float *r, const uint16_t *w, float eps, int32_t H, uint16_t *n) {
  float part[256];
  for (int j = 0; j < 256; ++j) {
    float p = 0.0f;
    for (int32_t c = j; c * 8 < H; c += 256)
      for (int32_t i = 8 * c; i < 8 * c + 8; ++i) p = p + r[i] * r[i];
    part[j] = p;
  }
  float g[4];
  for (int q = 0; q < 4; ++q) {
    float lane[ORC_LANES];
    for (int j = 0; j < ORC_LANES; ++j) lane[j] = part[q * ORC_LANES + j];
    for (int off = 1; off < ORC_LANES; off <<= 1) {
      float next[ORC_LANES];
      for (int j = 0; j < ORC_LANES; ++j) next[j] = lane[j] + lane[j ^ off];
      for (int j = 0; j < ORC_LANES; ++j) lane[j] = next[j];
    }
    g[q] = lane[0];
  }
  const float total = (g[0] + g[1]) + (g[2] + g[3]);
  const float inv = 1.0f / sqrtf(total / (float)H + eps);
  for (int32_t i = 0; i < H; ++i) n[i] = tobf(bf(w[i]) * bf(tobf(r[i] * inv)));
}

int orc_add_rms_norm(const uint16_t *h, const uint16_t *a, const uint16_t *w, float eps, int32_t T,
                     int32_t H, uint16_t *r_out, uint16_t *n_out) {
  if (T < 0 || H <= 0 || H % 8 != 0) return ORC_ERR_GEOMETRY;
  int err = ORC_OK;
#pragma omp parallel num_threads(g_threads)
  {
    float *r = (float *)malloc(sizeof(float) * (size_t)H);
    if (!r) {
#pragma omp atomic write
      err = ORC_ERR_GEOMETRY;
    } else {
#pragma omp for schedule(static)
      for (int32_t t = 0; t < T; ++t) {
        const size_t o = (size_t)t * H;
        for (int32_t i = 0; i < H; ++i) {
          float v = bf(h[o + i]);
          if (a) v = bf(tobf(v + bf(a[o + i])));
          r[i] = v;
          if (r_out) r_out[o + i] = tobf(v);
        }
        rms_norm_row(r, w, eps, H, n_out + o);
      }
    }
    free(r);
  }
  return err;
}

int orc_decoder_ffn_forward(const orc_layer *L, const uint16_t *h, const uint16_t *a, const uint16_t *w,
                            float eps, int32_t T, uint16_t *out, uint16_t *r_out) {
  const int32_t H = L->hidden;
  uint16_t *r = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * H + 2);
  uint16_t *n = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * H + 2);
  uint16_t *y = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * H + 2);
  int rc = (r && n && y) ? ORC_OK : ORC_ERR_GEOMETRY;
  if (!rc) rc = orc_add_rms_norm(h, a, w, eps, T, H, r, n);
  if (!rc) rc = orc_moe_block_forward(L, n, T, NULL, y, NULL);
  if (!rc) {
    for (size_t i = 0; i < (size_t)T * H; ++i) out[i] = tobf(bf(r[i]) + bf(y[i]));
    if (r_out) memcpy(r_out, r, sizeof(uint16_t) * (size_t)T * H);
  }
  free(r);
  free(n);
  free(y);
  return rc;
}

/*
 * Laguna's sigmoid router: select_laguna_router_experts (laguna/moe/router_selection.rs:59-116),
 * the reference's own CPU restatement of route_laguna_experts (laguna/moe/router.rs:29-94).
 * Per token: l = fp32 logit, l = tanh(l / c) * c when the softcap c > 0, s = sigmoid(l),
 * selection key s + bias; experts sorted by key descending (f32 total order) with the lower
 * expert id first on ties; the first k in that order; their unbiased s, divided by the
 * in-order fp32 sum when normalize and the sum is positive.  exp is orc_expf (the device's
 * det_expf bit for bit); tanh(x) = sign(x) (1 - 2 / (e^(2|x|) + 1)) on it.
 */
static float tanh_det(float x) {
  const float t = 1.0f - 2.0f / (orc_expf(2.0f * fabsf(x)) + 1.0f);
  return x != x ? x : copysignf(t, x);
}

static uint32_t total_order_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

int orc_laguna_route(const uint16_t *logits, int32_t T, int32_t E, int32_t k, const float *bias,
                     float softcap, int32_t normalize, uint32_t *indices, float *scores) {
  if (T < 0 || E <= 0 || k <= 0 || k > E || !(softcap >= 0.0f)) return ORC_ERR_GEOMETRY;
  uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)E);
  float *s = (float *)malloc(sizeof(float) * (size_t)E);
  if (!keys || !s) {
    free(keys);
    free(s);
    return ORC_ERR_GEOMETRY;
  }
  for (int32_t t = 0; t < T; ++t) {
    for (int32_t e = 0; e < E; ++e) {
      float l = bf(logits[(size_t)t * E + e]);
      if (softcap > 0.0f) l = tanh_det(l / softcap) * softcap;
      s[e] = sigmoidf_det(l);
      const float sel = s[e] + (bias ? bias[e] : 0.0f);
      keys[e] = ((uint64_t)total_order_bits(sel) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
    }
    /* k selections of the largest remaining key: descending key = descending score, lower id first */
    float sum = 0.0f;
    for (int32_t j = 0; j < k; ++j) {
      int32_t best = 0;
      for (int32_t e = 1; e < E; ++e)
        if (keys[e] > keys[best]) best = e;
      indices[(size_t)t * k + j] = (uint32_t)best;
      scores[(size_t)t * k + j] = s[best];
      sum = sum + s[best];
      keys[best] = 0;
    }
    if (normalize && sum > 0.0f)
      for (int32_t j = 0; j < k; ++j) scores[(size_t)t * k + j] = scores[(size_t)t * k + j] / sum;
  }
  free(keys);
  free(s);
  return ORC_OK;
}
