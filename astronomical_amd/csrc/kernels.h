// Internal launch interface of the gfx950 kernels (host side of each .hip file).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace astro {

// Rows of one grouped-GEMM tile; also the row granularity of the tile table the sort
// kernels emit.
constexpr int kGemmBM = 64;
// rows per tile of the exact-code GEMM, at most (the sort's second tile table splits every
// expert's rows into ceil(rows / kXqRows) tiles of balanced sizes)
constexpr int kXqRows = 80;

enum BKind { kBQ4 = 0, kBQ8 = 1, kBDense = 2 };
enum Epilogue { kEpiPlain = 0, kEpiSwiglu = 1, kEpiBias = 2 };

// out[dst(r)][n] = epilogue( sum_k A[src(r)][k] * B[expert(r)][n][k] ) over the rows r of
// every tile.  Tiles come from the tile table (expert, first row) written by the sort,
// or, when tile_expert == nullptr, from one implicit group of M rows.
struct GemmArgs {
  const uint16_t *A;
  int64_t lda;
  const uint32_t *a_rows;  // sorted row -> source index (nullptr: identity)
  int a_div;               // source row = a_rows[r] / a_div
  const uint32_t *a_rows2; // optional second indirection: source row = a_rows2[that]
  int K;
  int N;                   // output columns (activated columns for the SwiGLU epilogue)
  int bkind;
  // affine weights: gate (or the only projection) and, for SwiGLU, up
  const uint32_t *w0, *w1;
  const uint16_t *s0, *s1, *b0, *b1;
  int64_t w_expert_stride, w_row_stride;    // in u32 words
  int64_t sb_expert_stride, sb_row_stride;  // in bf16 elements
  int group;
  // dense bf16 weights [N][K]
  const uint16_t *bd;
  int64_t bd_row_stride;
  const uint16_t *bias;    // kEpiBias: bf16 [N]
  // tiles
  const uint32_t *tile_expert;
  const uint32_t *tile_row0;
  const uint32_t *tile_count;
  const uint32_t *expert_offsets;
  int M;                   // rows of the implicit single group
  int max_tiles;
  // output
  uint16_t *C;
  int64_t ldc;
  const uint32_t *c_rows;  // sorted row -> destination row (nullptr: identity)
  // optional fp32 group sums of the activation rows, xsum[src][gi] = sum of inputs gi * group ..
  // + group of source row src (launch_group_sums): 4-bit weights then run with exact codes
  const float *xsum;
  int64_t xsum_ld;
  int a_paired;  // the activation rows hold inputs (0, 4), (1, 5), (2, 6), (3, 7) of every 8
  // exact-code GEMM: the sort's table of balanced tiles of up to kXqRows rows (launch_sort's
  // xtiles, with room for max_xtiles entries)
  const uint32_t *xtiles;
  int max_xtiles;
  // exact-code SwiGLU epilogue: store the activated rows in the codes' pairing and the fp32
  // sums of their groups of c_group columns (c_xsum[row][group], row stride c_xsum_ld): the
  // a_paired / xsum inputs of an exact-code down projection
  int c_paired;
  float *c_xsum;
  int64_t c_xsum_ld;
  int c_group;
};

hipError_t launch_grouped_gemm(const GemmArgs &a, int epilogue, hipStream_t s);
// the exact-code grouped GEMM for 4-bit weights (gemm_xq.hip): a.xsum set, shapes it serves
bool xq_supported(const GemmArgs &a);
hipError_t launch_xq(const GemmArgs &a, const GemmArgs *b, int epilogue, hipStream_t s);
// X[r][gi] = fp32 sum of inputs gi * group .. + group of row r of A (rows x K bf16); paired
// (nullable, rows x K): the rows with inputs (0, 4), (1, 5), (2, 6), (3, 7) of every 8 paired
hipError_t launch_group_sums(const uint16_t *A, int64_t lda, int rows, int K, int group, float *X, int64_t ldx,
                             uint16_t *paired, hipStream_t s);
// a and, when b is non-null, a second problem b with the same epilogue in one launch (its
// tiles follow a's); problems the same kernel cannot serve are launched one after the other
hipError_t launch_grouped_gemm2(const GemmArgs &a, const GemmArgs *b, int epilogue, hipStream_t s);

// Affine weights over one implicit group of rows with exact codes on the MFMA (no bf16
// rounding of dequantised weights): the prefill router projection of an affine router.
bool affine_rows_supported(const GemmArgs &a, int epilogue);
hipError_t launch_affine_rows(const GemmArgs &a, int epilogue, hipStream_t s);

// Work on the token rows x (T rows of H) that the route kernel's wave per token also does:
// x's group sums and paired copy (the exact-code gate/up's inputs, as launch_group_sums writes
// them, groups of g; xsum null: not written) and the shared expert's output gate z (one affine
// row, as launch_qgemv_rows computes it; z null: not computed).  x null: neither.
struct RouteExtras {
  const uint16_t *x = nullptr;
  int H = 0, g = 0;
  float *xsum = nullptr;       // [T][H / g]
  uint16_t *paired = nullptr;  // [T][H]
  const uint32_t *zw = nullptr;
  const uint16_t *zs = nullptr, *zb = nullptr;
  int zbits = 0, zgroup = 0;
  uint16_t *z = nullptr;       // [T]
};
hipError_t launch_route_topk(const uint16_t *logits, int T, int E, int k, int normalize,
                             uint32_t *idx, uint16_t *scores, hipStream_t s,
                             const RouteExtras &ex = RouteExtras());

// counting sort of assignment ids by expert (stable), plus the grouped-GEMM tile table
// (tiles of kGemmBM rows).  offsets has E+2 entries (ids >= E land in a trailing
// bucket that no tile covers).  With xtiles set, also the exact-code GEMM's table
// (2 + 2 * sort_max_xtiles(A, E) words): word 0 the tile count, then per tile
// (expert | rows << 16, first sorted row), experts ascending.
// scratch: sort_scratch_bytes(A, E) bytes (per-chunk histograms and local ranks)
hipError_t launch_sort(const uint32_t *ids, int A, int E, uint32_t *sorted_order,
                       uint32_t *inverse_order, uint32_t *sorted_ids, uint32_t *offsets,
                       uint32_t *tile_expert, uint32_t *tile_row0, uint32_t *tile_count,
                       uint32_t *scratch, hipStream_t s, uint32_t *xtiles = nullptr);
size_t sort_scratch_bytes(int A, int E);
int sort_max_tiles(int A, int E);
int sort_max_xtiles(int A, int E);

// out[t] = bf16( x[t] . deq(W row n) ) for a few output rows (wave per (token, row)).
hipError_t launch_qgemv_rows(const uint16_t *x, int T, int K, const uint32_t *w,
                             const uint16_t *sc, const uint16_t *bi, int N, int bits, int group,
                             uint16_t *out, hipStream_t s);

// Multi-token quantized linear (target-verification windows and small-batch quantized
// matmul): y[m] = x[m] . deq(W)^T for M token rows, bf16 or f16 activations / scales /
// biases / outputs, 4-, 5- or 8-bit codes.  One launch per kVerifyRows rows; every output
// has the bits it has at M = 1.
constexpr int kVerifyRows = 16;
bool verify_qmv_supported(int K, int bits, int group, const void *x, const void *w);
hipError_t launch_verify_qmv(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc,
                             const uint16_t *bi, int N, int bits, int group, bool f16, uint16_t *y,
                             hipStream_t s);

hipError_t launch_swiglu(const uint16_t *g, const uint16_t *u, int64_t n, uint16_t *out,
                         hipStream_t s);

// paged callers: slots[a] = slot_of_expert[ids[a]] (absent experts count into *missing and
// read slot 0); assignment gather by position; bf16 add
hipError_t launch_remap_slots(const uint32_t *ids, int n, const uint32_t *slot_of_expert, int experts,
                              uint32_t *slots, uint32_t *missing, hipStream_t s);
hipError_t launch_gather_assignments(const uint32_t *ids, const uint16_t *scores,
                                     const uint32_t *positions, int n, uint32_t *out_ids,
                                     uint16_t *out_scores, hipStream_t s);
hipError_t launch_add_bf16(const uint16_t *a, const uint16_t *b, int64_t n, uint16_t *out, hipStream_t s);
// *count = the fp32 bit patterns (all 2^32) whose f2bf differs from f2bf_bits
hipError_t launch_selftest_bf16(unsigned long long *count, hipStream_t s);
hipError_t launch_zero_u32(uint32_t *p, int n, hipStream_t s);  // a kernel, safe in graph capture
// decoder step around the block: r = bf16(h + a) (a nullable; r_out nullable), n = RMSNorm(r)
// with weight w (H <= 8192)
hipError_t launch_add_rms_norm(const uint16_t *h, const uint16_t *a, const uint16_t *w, float eps, int T,
                               int H, uint16_t *r_out, uint16_t *n_out, hipStream_t s);
// Laguna's sigmoid router (E <= 1024, k <= 64): idx u32 [T][k], fp32 scores [T][k]
hipError_t launch_route_laguna(const uint16_t *logits, int T, int E, int k, const float *bias, float softcap,
                               int normalize, uint32_t *idx, float *scores, hipStream_t s);
// y = weighted sum of expert rows (rows located through inverse_order), sorted (fp32
// fma accumulation) or unsorted (bf16 products) rounding, then optionally the shared
// expert's gated add.
hipError_t launch_combine(const uint16_t *rows, const uint32_t *inverse_order,
                          const uint16_t *scores, int T, int k, int D, int sorted,
                          const uint16_t *shared_out, const uint16_t *gate_logits,
                          uint16_t *sparse_out, uint16_t *y, hipStream_t s);
hipError_t launch_combine_shared(const uint16_t *sparse, const uint16_t *shared_out,
                                 const uint16_t *gate_logits, int T, int D, uint16_t *y,
                                 hipStream_t s);

// Decode path (T <= 8 tokens, T*k <= 64): every pointer is a device pointer; rows of `act`
// and `down_out` are the A sorted assignments followed by the T shared-expert rows.
struct DecodeArgs {
  int T, A, H, E, k, I, Is, normalize;
  const uint16_t *x, *router_w, *router_bias;
  // affine router (router_w null): codes [E][H * rq_bits / 32], scales / biases [E][H / rq_group]
  const uint32_t *rq_w;
  const uint16_t *rq_s, *rq_b;
  int rq_bits, rq_group;
  int64_t rq_w_rs, rq_sb_rs;
  // routed gate/up (fused or separate pages share strides) and down
  const uint32_t *gate_w, *up_w, *down_w;
  const uint16_t *gate_s, *gate_b, *up_s, *up_b, *down_s, *down_b;
  int64_t gu_w_es, gu_w_rs, gu_sb_es, gu_sb_rs;
  int64_t dn_w_es, dn_w_rs, dn_sb_es, dn_sb_rs;
  int gu_bits, gu_group, dn_bits, dn_group;
  // shared expert
  const uint32_t *sg_w, *su_w, *sd_w, *sz_w;
  const uint16_t *sg_s, *sg_b, *su_s, *su_b, *sd_s, *sd_b, *sz_s, *sz_b;
  int64_t sg_w_rs, sg_sb_rs, sd_w_rs, sd_sb_rs;
  int sg_bits, sg_group, sd_bits, sd_group, sz_bits, sz_group;
  // workspace
  uint16_t *logits, *scores;
  uint32_t *idx, *sorted_order, *inverse_order, *sorted_ids, *offsets;
  uint32_t *n_groups, *g_expert, *g_start, *g_count;
  uint32_t *g_tokens;  // [64][kDecodeMaxK]: the tokens of group g's sorted rows (the last repeated)
  uint16_t *act, *down_out, *z;
  int64_t act_ld;
  uint16_t *sparse, *y;  // outputs: weighted sum of the routed experts, block output
  int router_blocks, shared_pair_blocks, max_groups;
  // decoder step (norm_w set): the router kernel forms r = bf16(h_in + a_in) (a_in nullable)
  // and the RMS-normalised rows itself (its first workgroup writes them to r_out and x_out; x
  // must be x_out), and the down kernel also writes ffn_out = bf16(r + y)
  const uint16_t *h_in, *a_in, *norm_w;
  float eps;
  uint16_t *r_out, *x_out, *ffn_out;
  // target-verification windows: the unsorted combine at every A (token-local rows)
  bool unsorted;
  // compact pages (slot_of_expert set, [E]): an expert's weights are at its page slot, the
  // assignments sort by slot (buckets: max(E, the page's slot count)); an expert with no slot
  // (0xffffffff) reads slot 0 and is counted in *missing (remap_slots_kernel's rule); slots[a]
  // = the slot of assignment a; a slot past the page (>= slot_count) is treated as absent
  const uint32_t *slot_of_expert;
  uint32_t *slots, *missing;
  int buckets, slot_count;
};
// the router kernel keeps the T normalised rows in LDS: the decoder step fuses into the decode
// kernels when T * H * 2 bytes fit
constexpr int kDecodeStepLds = 60 * 1024;

bool decode_supported(const DecodeArgs &a);
constexpr int kDecodeRowsPerWave = 1;  // must match kRowsPerWave in decode.hip
// from this many tokens a one-workgroup kernel routes the batch once, instead of every routed
// gate/up workgroup recomputing every token's top-k set (one wave per token; c1: B = 2 23.6 us
// per layer in-workgroup against 24.3 with the routing kernel, B = 4 33.7 against 33.1)
constexpr int kDecodeRouteOnceT = 3;
constexpr int kDecodeMaxK = 8;         // experts per token the decode combine unrolls
// the down kernel's output rows per quarter-wave: 1 up to kDecodeDownR1T tokens, 2 up to
// kDecodeDownR2T, then 4
constexpr int kDecodeDownR1T = 1;
constexpr int kDecodeDownR2T = 2;
// the down kernel's workgroup takes one wave per participant up to this many tokens (c1: B = 1
// 17.0 -> 16.3, B = 4 33.3 -> 31.2 us per layer), then 3 waves of 3 (B = 8: 48.1 against 49.4)
constexpr int kDecodeDownWideT = 4;
// tokens per pass of a gate/up wave of several row pairs (fewer registers, more waves per SIMD)
constexpr int kDecodePassTokens = 2;
// launches the decode kernels (router | [routing, T >= kDecodeRouteOnceT] | shared gate/up +
// routing (T = 1) + routed gate/up | down + combine); kev (nullable) = start/stop event pairs
// recorded around the router, gate/up and down kernels, and (kev[6..7]) the routing kernel
hipError_t launch_decode_block(const DecodeArgs &a, hipStream_t s, const hipEvent_t *kev);

}  // namespace astro
