// Host layer of the C ABI: argument validation (mirroring the reference's checks and
// messages), the workspace layout, and the launch sequence of the block.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/astro_moe.h"
#include "kernels.h"
#include "status.h"

using namespace astro;

namespace {

int fail(int status, const char *op, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int fail(int status, const char *op, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int r = vreport(status, op, fmt, ap);
  va_end(ap);
  return r;
}

int ok() { return report_ok(); }

int hip_fail(const char *op, hipError_t e) {
  return fail(ASTRO_MOE_HIP_ERROR, op, "HIP error %d (%s)", (int)e, hipGetErrorString(e));
}

// The marker keeps classify_mlx_error (error_handling.rs:81-122) classifying the failure
// as ActiveMemoryLimitExceeded; only key=value fields may follow it.
int workspace_fail(const char *op, size_t need, size_t have) {
  return fail(ASTRO_MOE_WORKSPACE_TOO_SMALL, op,
              "ASTRONOMICAL_MLX_ACTIVE_MEMORY_LIMIT_EXCEEDED active_bytes=0 allocation_bytes=%zu "
              "allowed_bytes=%zu",
              need, have);
}

}  // namespace


namespace {

const char *const kBlockOp = "run the Qwen3.5-MoE sparse expert block";
const char *const kRouteOp = "route Qwen3.5-MoE sparse experts";           // routing.rs:11
const char *const kSortOp = "sort stacked expert assignments";             // assignment_sort.rs:10
const char *const kReduceOp = "reduce stacked expert outputs";             // weighted_sum.rs:15
const char *const kCombineOp = "combine Qwen3.5-MoE sparse and shared experts";  // routing.rs:12
const char *const kGatherOp = "build affine gather_qmm";                  // mlx_quantized_operations.rs:114
const char *const kQmmOp = "build affine quantized matmul";               // mlx_quantized_operations.rs:60
const char *const kPermOp = "invert assignment permutation";

// validate_affine_quantized_matmul_arguments (mlx_quantized_operations.rs:226-330), then
// what the gfx950 kernels implement.
int check_affine(const char *op, const astro_moe_affine *w, int inner) {
  if (!w || !w->w || !w->scales || !w->biases)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "affine weights, scales and biases must be non-null");
  if (w->group_size != 32 && w->group_size != 64 && w->group_size != 128)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "affine group size must be 32, 64, or 128");
  if (w->bits != 2 && w->bits != 3 && w->bits != 4 && w->bits != 5 && w->bits != 6 && w->bits != 8)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "affine bit width must be 2, 3, 4, 5, 6, or 8");
  if (w->experts <= 0 || w->out_features <= 0 || w->in_features <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "array shape must have a positive tail dimension");
  if (((int64_t)w->in_features * w->bits) % 32 != 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "packed weight shape overflows or is incompatible with the requested bit width");
  if (w->in_features % w->group_size != 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "affine scale and bias shapes do not match the packed weight shape");
  if (inner >= 0 && inner != w->in_features)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "activation inner dimension does not match the expanded quantized weight input");
  if (w->bits != 4 && w->bits != 8)
    return fail(ASTRO_MOE_UNSUPPORTED, op, "the gfx950 kernels implement 4-bit and 8-bit affine weights");
  if (w->in_features % 64 != 0)
    return fail(ASTRO_MOE_UNSUPPORTED, op, "the gfx950 kernels need an input width that is a multiple of 64");
  return ASTRO_MOE_OK;
}

int64_t words_per_row(const astro_moe_affine &w) { return (int64_t)w.in_features * w.bits / 32; }
int64_t groups_per_row(const astro_moe_affine &w) { return w.in_features / w.group_size; }

// Fill the weight part of a GemmArgs from one projection (or a gate/up pair).
void set_weights(GemmArgs &g, const astro_moe_affine &gate, const astro_moe_affine *up,
                 int64_t up_row_offset) {
  g.bkind = gate.bits == 8 ? kBQ8 : kBQ4;
  g.group = gate.group_size;
  g.w_row_stride = words_per_row(gate);
  g.sb_row_stride = groups_per_row(gate);
  g.w_expert_stride = (int64_t)gate.out_features * g.w_row_stride;
  g.sb_expert_stride = (int64_t)gate.out_features * g.sb_row_stride;
  g.w0 = gate.w;
  g.s0 = gate.scales;
  g.b0 = gate.biases;
  if (up) {
    g.w1 = up->w + up_row_offset * g.w_row_stride;
    g.s1 = up->scales + up_row_offset * g.sb_row_stride;
    g.b1 = up->biases + up_row_offset * g.sb_row_stride;
  }
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

struct Layout {
  size_t logits, idx, scores, sorted_order, inverse, sorted_ids, offsets, tile_expert, tile_row0,
      tile_count, act, eout, sparse, shared_act, shared_out, z, groups, sort_scratch, slots, missing,
      xsum_x, xsum_act, xsum_sact, xpair, xtiles, total;
  int max_tiles, max_xtiles;
  bool decode;     // wavefront-GEMV path: act / eout hold A routed rows then T shared rows
  int64_t act_ld;  // row length of act
};

// The decode path takes small batches: at most 8 tokens and 64 assignments, a bf16 or affine
// router, resident experts or a compact page, and shapes its per-lane register tiles cover
// (decode.hip: decode_supported).
// Leading dimension of the routed expert arrays: the expert count for resident weights, the
// page's slot count for compact pages (slot_of_expert set).
int expert_capacity(const astro_moe_layer &L) {
  return L.gate_up.w ? L.gate_up.experts : L.gate.experts;
}

bool decode_path(const astro_moe_layer &L, int T) {
  const int Is = L.shared_intermediate > 0 ? L.shared_intermediate : 0;
  const astro_moe_affine &gu = L.gate_up.w ? L.gate_up : L.gate;
  const bool router_ok = L.router_w ? true
                                    : (L.router_q.bits == 4 || L.router_q.bits == 8) && L.router_q.group_size >= 32;
  return T >= 1 && T <= 8 && T * L.top_k <= 64 && L.top_k <= kDecodeMaxK &&
         router_ok && L.hidden <= 4096 &&
         L.intermediate <= 1024 && Is <= 1024 && (gu.bits == 4 || gu.bits == 8) &&
         (L.down.bits == 4 || L.down.bits == 8) &&
         (Is == 0 || L.shared_down.bits == L.down.bits);
}

// Workspace of the block (kk = top_k) or of the streamed sparse forward (kk = assignments per
// token, no routing and no shared expert: with_router = false).
Layout block_layout(const astro_moe_layer &L, int T, int kk, bool with_router) {
  Layout o{};
  const size_t A = (size_t)T * kk;
  // ids the sort buckets: expert ids, or page slots
  const size_t E = (size_t)std::max(L.num_experts, expert_capacity(L));
  const size_t Is = with_router && L.shared_intermediate > 0 ? (size_t)L.shared_intermediate : 0;
  o.decode = with_router && decode_path(L, T);
  o.max_tiles = o.decode ? 0 : sort_max_tiles((int)A, (int)E);
  size_t p = 0;
  auto take = [&](size_t bytes) {
    const size_t at = p;
    p = align_up(p + bytes);
    return at;
  };
  o.logits = take(with_router ? (size_t)T * L.num_experts * 2 : 0);
  o.idx = take(A * 4);
  o.scores = take(A * 2);
  o.sorted_order = take(A * 4);
  o.inverse = take(A * 4);
  o.sorted_ids = take(A * 4);
  o.offsets = take((E + 2) * 4);
  if (o.decode) {
    // n_groups, then expert / first row / count of up to 64 groups
    o.groups = take(4 + 3 * 64 * 4 + 64 * kDecodeMaxK * 4);  // count, expert / start / rows, tokens
    o.act_ld = std::max<int64_t>(L.intermediate, (int64_t)Is);
    o.act = take((A + (Is ? T : 0)) * (size_t)o.act_ld * 2);
    o.eout = take((A + (Is ? T : 0)) * (size_t)L.hidden * 2);
    o.sparse = take((size_t)T * L.hidden * 2);
    o.shared_out = Is ? o.eout + A * (size_t)L.hidden * 2 : 0;
    o.z = take(Is ? (size_t)T * 2 : 0);
    o.slots = take(L.slot_of_expert ? A * 4 : 0);
    o.missing = take(L.slot_of_expert ? 4 : 0);
  } else {
    o.tile_expert = take((size_t)o.max_tiles * 4);
    o.tile_row0 = take((size_t)o.max_tiles * 4);
    o.tile_count = take(4);
    o.sort_scratch = take(sort_scratch_bytes((int)A, (int)E));
    o.act_ld = L.intermediate;
    o.act = take(A * (size_t)L.intermediate * 2);
    o.eout = take(A * (size_t)L.hidden * 2);
    o.sparse = take((size_t)T * L.hidden * 2);
    o.shared_act = take((size_t)T * Is * 2);
    o.shared_out = take(Is ? (size_t)T * L.hidden * 2 : 0);
    o.z = take(Is ? (size_t)T * 2 : 0);
    o.slots = take(with_router && L.slot_of_expert ? A * 4 : 0);
    o.missing = take(with_router && L.slot_of_expert ? 4 : 0);
    // fp32 group sums of x, of the activated rows and of the shared expert's activated rows
    // (the exact-code GEMMs' affine terms), sized for groups of 32
    o.xsum_x = take((size_t)T * (L.hidden / 32) * 4);
    o.xpair = take((size_t)T * L.hidden * 2);
    o.xsum_act = take(A * (size_t)(L.intermediate / 32) * 4);
    o.xsum_sact = take((size_t)T * (Is / 32) * 4);
    // the exact-code GEMMs' table of balanced tiles (launch_sort)
    o.max_xtiles = sort_max_xtiles((int)A, (int)E);
    o.xtiles = take((2 + 2 * (size_t)o.max_xtiles) * 4);
  }
  o.total = p;
  return o;
}

// The routed expert arrays: fused gate/up or separate gate and up, and down, all with
// `capacity` experts (the expert count, or a compact page's slots).
int check_routed(const char *op, const astro_moe_layer *L, int capacity) {
  const int H = L->hidden, I = L->intermediate;
  if (capacity <= 0 || capacity > 1024)
    return fail(ASTRO_MOE_UNSUPPORTED, op, "expert arrays must hold between 1 and 1024 experts or page slots");
  if (H % 64 != 0 || I % 64 != 0)
    return fail(ASTRO_MOE_UNSUPPORTED, op, "the gfx950 kernels need hidden and intermediate sizes that are multiples of 64");
  if (L->gate_up.w) {
    int rc = check_affine(op, &L->gate_up, H);
    if (rc) return rc;
    if (L->gate_up.experts != capacity || L->gate_up.out_features != 2 * I)
      return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "resident fused gate/up output dimension must be twice the intermediate size");
  } else {
    int rc = check_affine(op, &L->gate, H);
    if (!rc) rc = check_affine(op, &L->up, H);
    if (rc) return rc;
    if (L->gate.experts != capacity || L->up.experts != capacity || L->gate.out_features != I ||
        L->up.out_features != I || L->gate.bits != L->up.bits || L->gate.group_size != L->up.group_size)
      return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "separate gate and up projections must share shape and quantization");
  }
  int rc = check_affine(op, &L->down, I);
  if (rc) return rc;
  if (L->down.experts != capacity || L->down.out_features != H)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "down projection must map the intermediate size back to the hidden size");
  return ASTRO_MOE_OK;
}

int check_layer(const char *op, const astro_moe_layer *L) {
  if (!L) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "layer description must be non-null");
  const int H = L->hidden, E = L->num_experts, k = L->top_k, I = L->intermediate;
  if (H <= 0 || E <= 0 || I <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "hidden, expert and intermediate sizes must be positive");
  if (k <= 0 || k > E)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "selected expert count must be positive and no larger than the router dimension");
  if (E > 1024 || k > 64)
    return fail(ASTRO_MOE_UNSUPPORTED, op, "the router kernel supports at most 1024 experts and top-64");
  if (!!L->router_w == !!L->router_q.w)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "exactly one of the dense and affine router weights must be set");
  if (L->router_q.w) {
    int rc = check_affine(op, &L->router_q, H);
    if (rc) return rc;
    if (L->router_q.experts != 1 || L->router_q.out_features != E)
      return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "router weights must map the hidden size to the expert count");
  }
  {
    // resident arrays hold every expert; a compact page (slot_of_expert set) any slot count
    const astro_moe_affine &first = L->gate_up.w ? L->gate_up : L->gate;
    int rc = check_routed(op, L, L->slot_of_expert ? first.experts : E);
    if (rc) return rc;
  }
  if (L->shared_intermediate < 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "shared expert intermediate size must not be negative");
  if (L->shared_intermediate > 0) {
    const int Is = L->shared_intermediate;
    int rc = check_affine(op, &L->shared_gate, H);
    if (!rc) rc = check_affine(op, &L->shared_up, H);
    if (!rc) rc = check_affine(op, &L->shared_down, Is);
    if (!rc) rc = check_affine(op, &L->shared_expert_gate, H);
    if (rc) return rc;
    if (Is % 64 != 0)
      return fail(ASTRO_MOE_UNSUPPORTED, op, "the gfx950 kernels need a shared intermediate size that is a multiple of 64");
    if (L->shared_gate.out_features != Is || L->shared_up.out_features != Is ||
        L->shared_down.out_features != H || L->shared_expert_gate.out_features != 1 ||
        L->shared_gate.bits != L->shared_up.bits || L->shared_gate.group_size != L->shared_up.group_size)
      return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "shared expert projections have inconsistent shapes");
  }
  return ASTRO_MOE_OK;
}

hipError_t run_router(const astro_moe_layer &L, const uint16_t *x, int T, uint16_t *logits,
                      hipStream_t s) {
  GemmArgs g{};
  g.A = x;
  g.lda = L.hidden;
  g.a_div = 1;
  g.K = L.hidden;
  g.N = L.num_experts;
  g.M = T;
  g.C = logits;
  g.ldc = L.num_experts;
  if (L.router_w) {
    g.bkind = kBDense;
    g.bd = L.router_w;
    g.bd_row_stride = L.hidden;
  } else {
    set_weights(g, L.router_q, nullptr, 0);
  }
  g.bias = L.router_bias;
  const int epi = L.router_bias ? kEpiBias : kEpiPlain;
  // an affine router keeps its codes exact (the routing bits hang on the logits)
  if (!L.router_w && affine_rows_supported(g, epi)) return launch_affine_rows(g, epi, s);
  return launch_grouped_gemm(g, epi, s);
}

// shared expert problems: act = swiglu(gate(x), up(x)) (gu); out = down(act) (dn)
void shared_gemm_args(const astro_moe_layer &L, const uint16_t *x, int T, uint16_t *act,
                      uint16_t *out, GemmArgs &gu, GemmArgs &dn) {
  gu = GemmArgs{};
  gu.A = x;
  gu.lda = L.hidden;
  gu.a_div = 1;
  gu.K = L.hidden;
  gu.N = L.shared_intermediate;
  gu.M = T;
  set_weights(gu, L.shared_gate, &L.shared_up, 0);
  gu.w_expert_stride = gu.sb_expert_stride = 0;
  gu.C = act;
  gu.ldc = L.shared_intermediate;
  dn = GemmArgs{};
  dn.A = act;
  dn.lda = L.shared_intermediate;
  dn.a_div = 1;
  dn.K = L.shared_intermediate;
  dn.N = L.hidden;
  dn.M = T;
  set_weights(dn, L.shared_down, nullptr, 0);
  dn.C = out;
  dn.ldc = L.hidden;
}

hipError_t run_shared_gate(const astro_moe_layer &L, const uint16_t *x, int T, uint16_t *z,
                           hipStream_t s) {
  const astro_moe_affine &zg = L.shared_expert_gate;
  return launch_qgemv_rows(x, T, L.hidden, zg.w, zg.scales, zg.biases, 1, zg.bits, zg.group_size,
                           z, s);
}

// shared expert: act = swiglu(gate(x), up(x)); out = down(act); z = shared_expert_gate(x)
hipError_t run_shared(const astro_moe_layer &L, const uint16_t *x, int T, uint16_t *act,
                      uint16_t *out, uint16_t *z, hipStream_t s) {
  GemmArgs gu, dn;
  shared_gemm_args(L, x, T, act, out, gu, dn);
  hipError_t e = launch_grouped_gemm(gu, kEpiSwiglu, s);
  if (e == hipSuccess) e = launch_grouped_gemm(dn, kEpiPlain, s);
  if (e == hipSuccess) e = run_shared_gate(L, x, T, z, s);
  return e;
}

// Per-stage device times for the attributed entry point: a start and a stop event per
// stage (router, route, sort, gate/up, down, shared, combine).  Kernels that make up a
// stage on their own are launched with the events attached to the kernel itself
// (hipExtLaunchKernelGGL), other stages are bracketed by event records; stages with no
// work of their own (routing inside the decode gate/up kernel, for one) stay unused.
struct StageClock {
  hipEvent_t *ev;  // 2 * ASTRO_MOE_STAGES: start, stop
  hipStream_t s;
  bool used[ASTRO_MOE_STAGES];
  void begin(int i) {
    used[i] = true;
    (void)hipEventRecord(ev[2 * i], s);
  }
  void end(int i) { (void)hipEventRecord(ev[2 * i + 1], s); }
};

// The sparse graph after routing (forward_moe_with_streamed_weights, paged_execution.rs:207-281,
// and the resident arm of resident_execution.rs:70-143): sort the assignments by id (expert or
// page slot), gate/up with the SwiGLU epilogue over rows x[sorted_order[r] / kk], down, and the
// weighted sum -- sorted rounding iff A >= 64 (routing.rs:13) and not force_unsorted (an MTP
// verification window).  with_shared: the shared expert's gate/up and down run in the routed
// launches and y = the shared combine; otherwise y = the sparse output.
// The GEMM problems of the sorted path: routed gate/up (SwiGLU) and down, and the shared
// expert's, with the exact-code inputs decided: 4-bit gate/up reads x's copy in the codes'
// pairing with its group sums (paired_x); its epilogue then writes the activated rows paired,
// with their group sums, for an exact-code down projection (act_paired).  Neither happens when
// the exact-code kernel cannot take the problem.
struct SparsePlan {
  GemmArgs gu{}, dn{}, sgu{}, sdn{};
  bool has_shared = false;
  bool paired_x = false;    // x's group sums and paired copy are needed
  bool act_paired = false;  // the routed activated rows are stored in the codes' pairing
};

SparsePlan plan_sparse(const astro_moe_layer &L, const uint16_t *x, int T, int kk, const Layout &o, char *ws,
                       bool with_shared) {
  auto at = [&](size_t off) { return (void *)(ws + off); };
  SparsePlan P;
  const int H = L.hidden, I = L.intermediate;
  P.has_shared = with_shared && L.shared_intermediate > 0;
  const astro_moe_affine &gu_w = L.gate_up.w ? L.gate_up : L.gate;
  float *xs_x = (float *)at(o.xsum_x), *xs_act = (float *)at(o.xsum_act), *xs_sact = (float *)at(o.xsum_sact);
  uint32_t *offsets = (uint32_t *)at(o.offsets);
  // gate/up with the SwiGLU epilogue: rows gathered as x[sorted_order[r] / kk]
  GemmArgs &gu = P.gu;
  gu.A = x;
  gu.lda = H;
  gu.a_rows = (const uint32_t *)at(o.sorted_order);
  gu.a_div = kk;
  gu.K = H;
  gu.N = I;
  if (L.gate_up.w)
    set_weights(gu, L.gate_up, &L.gate_up, I);
  else
    set_weights(gu, L.gate, &L.up, 0);
  gu.tile_expert = (const uint32_t *)at(o.tile_expert);
  gu.tile_row0 = (const uint32_t *)at(o.tile_row0);
  gu.tile_count = (const uint32_t *)at(o.tile_count);
  gu.expert_offsets = offsets;
  gu.max_tiles = o.max_tiles;
  gu.xtiles = (const uint32_t *)at(o.xtiles);
  gu.max_xtiles = o.max_xtiles;
  gu.C = (uint16_t *)at(o.act);
  gu.ldc = I;
  GemmArgs &dn = P.dn;
  dn.A = (const uint16_t *)at(o.act);
  dn.lda = I;
  dn.a_div = 1;
  dn.K = I;
  dn.N = H;
  set_weights(dn, L.down, nullptr, 0);
  dn.tile_expert = gu.tile_expert;
  dn.tile_row0 = gu.tile_row0;
  dn.tile_count = gu.tile_count;
  dn.expert_offsets = offsets;
  dn.max_tiles = o.max_tiles;
  dn.xtiles = gu.xtiles;
  dn.max_xtiles = o.max_xtiles;
  dn.C = (uint16_t *)at(o.eout);
  dn.ldc = H;
  // the shared expert's gate/up and down run in the same launches as the routed ones
  if (P.has_shared)
    shared_gemm_args(L, x, T, (uint16_t *)at(o.shared_act), (uint16_t *)at(o.shared_out), P.sgu, P.sdn);
  auto paired_x = [&](GemmArgs &g) {
    GemmArgs t = g;
    t.xsum = xs_x;
    t.xsum_ld = H / gu_w.group_size;
    t.A = (const uint16_t *)at(o.xpair);
    t.lda = H;
    t.a_paired = 1;
    if (gu_w.bits == 4 && t.group == gu_w.group_size && xq_supported(t)) g = t;
  };
  auto paired_act = [&](GemmArgs &up, GemmArgs &down, float *sums) {
    if (!up.a_paired) return false;
    GemmArgs u = up, d = down;
    u.c_paired = 1;
    u.c_xsum = sums;
    u.c_xsum_ld = down.K / down.group;
    u.c_group = down.group;
    d.a_paired = 1;
    d.xsum = sums;
    d.xsum_ld = u.c_xsum_ld;
    if (!xq_supported(u) || !xq_supported(d)) return false;
    up = u;
    down = d;
    return true;
  };
  paired_x(gu);
  if (P.has_shared) paired_x(P.sgu);
  P.paired_x = gu.a_paired || (P.has_shared && P.sgu.a_paired);
  P.act_paired = paired_act(gu, dn, xs_act);
  if (P.has_shared) paired_act(P.sgu, P.sdn, xs_sact);
  return P;
}

hipError_t run_sparse(const astro_moe_layer &L, const uint16_t *x, int T, int kk, const uint32_t *ids,
                      const uint16_t *scores, const Layout &o, char *ws, bool with_shared, uint16_t *y,
                      hipStream_t s, StageClock *clock, bool force_unsorted = false, bool sums_ready = false,
                      bool gate_ready = false) {
  auto at = [&](size_t off) { return (void *)(ws + off); };
  auto begin = [&](int i) {
    if (clock) clock->begin(i);
  };
  auto end = [&](int i) {
    if (clock) clock->end(i);
  };
  const int H = L.hidden, A = T * kk;
  const int E = std::max(L.num_experts, expert_capacity(L));
  uint32_t *inverse = (uint32_t *)at(o.inverse);
  uint16_t *eout = (uint16_t *)at(o.eout);
  uint16_t *sparse = (uint16_t *)at(o.sparse);
  SparsePlan P = plan_sparse(L, x, T, kk, o, ws, with_shared);
  const bool has_shared = P.has_shared;
  GemmArgs &gu = P.gu, &dn = P.dn, &sgu = P.sgu, &sdn = P.sdn;
  uint16_t *shared_out = has_shared ? (uint16_t *)at(o.shared_out) : nullptr;
  uint16_t *z = has_shared ? (uint16_t *)at(o.z) : nullptr;
  const astro_moe_affine &gu_w = L.gate_up.w ? L.gate_up : L.gate;

  // the sort stage also takes x's group sums and paired copy (the exact-code gate/up's
  // inputs), so the gate/up stage is the one GEMM launch; sums_ready: the route kernel has
  // written them (gate_ready: and the shared expert's output gate z)
  begin(2);
  hipError_t e = launch_sort(ids, A, E, (uint32_t *)at(o.sorted_order), inverse, (uint32_t *)at(o.sorted_ids),
                             (uint32_t *)at(o.offsets), (uint32_t *)at(o.tile_expert), (uint32_t *)at(o.tile_row0),
                             (uint32_t *)at(o.tile_count), (uint32_t *)at(o.sort_scratch), s,
                             (uint32_t *)at(o.xtiles));
  if (e == hipSuccess && P.paired_x && !sums_ready)
    e = launch_group_sums(x, H, T, H, gu_w.group_size, (float *)at(o.xsum_x), H / gu_w.group_size,
                          (uint16_t *)at(o.xpair), s);
  end(2);
  if (e != hipSuccess) return e;
  begin(3);
  // the shared expert's tiles (whole tiles) first: the dispatcher deals workgroups in order, so
  // the lighter routed tiles fill the last, partial round of the grid
  e = has_shared ? launch_grouped_gemm2(sgu, &gu, kEpiSwiglu, s) : launch_grouped_gemm2(gu, nullptr, kEpiSwiglu, s);
  end(3);

  begin(4);
  if (e == hipSuccess)
    e = has_shared ? launch_grouped_gemm2(sdn, &dn, kEpiPlain, s) : launch_grouped_gemm2(dn, nullptr, kEpiPlain, s);
  end(4);

  if (has_shared && !gate_ready) {
    begin(5);
    if (e == hipSuccess) e = run_shared_gate(L, x, T, z, s);
    end(5);
  }
  begin(6);
  if (e == hipSuccess)
    e = launch_combine(eout, inverse, scores, T, kk, H, A >= 64 && !force_unsorted, shared_out, z, sparse, y, s);
  end(6);
  return e;
}

// The block's launch sequence; clock (nullable) collects per-stage times.
// The decoder step around the block (astro_moe_decoder_ffn_forward): x must be n; the decode
// kernels fuse r, n and out when the T rows fit their LDS, otherwise separate kernels run.
struct DecoderStep {
  const uint16_t *h, *a, *w;
  float eps;
  uint16_t *r, *n, *out;
};

int run_block(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens, uint16_t *y,
              void *workspace, size_t workspace_bytes, void *stream, StageClock *clock,
              const DecoderStep *step = nullptr, bool verification = false) {
  int rc = check_layer(kBlockOp, layer);
  if (rc) return rc;
  if (tokens < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "token count must not be negative");
  if (tokens == 0) return ok();
  if (!x || !y) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "hidden states and output must be non-null");
  const astro_moe_layer &L = *layer;
  const Layout o = block_layout(L, tokens, L.top_k, true);
  if (!workspace || workspace_bytes < o.total) return workspace_fail(kBlockOp, o.total, workspace ? workspace_bytes : 0);
  hipStream_t s = (hipStream_t)stream;
  char *ws = (char *)workspace;
  auto at = [&](size_t off) { return (void *)(ws + off); };
  const int T = tokens, H = L.hidden, E = L.num_experts, k = L.top_k, I = L.intermediate;
  const int A = T * k;
  uint16_t *logits = (uint16_t *)at(o.logits);
  uint32_t *idx = (uint32_t *)at(o.idx);
  uint16_t *scores = (uint16_t *)at(o.scores);
  uint32_t *sorted_order = (uint32_t *)at(o.sorted_order);
  uint32_t *inverse = (uint32_t *)at(o.inverse);
  uint32_t *sorted_ids = (uint32_t *)at(o.sorted_ids);
  uint32_t *offsets = (uint32_t *)at(o.offsets);
  uint32_t *tile_expert = (uint32_t *)at(o.tile_expert);
  uint32_t *tile_row0 = (uint32_t *)at(o.tile_row0);
  uint32_t *tile_count = (uint32_t *)at(o.tile_count);
  uint16_t *act = (uint16_t *)at(o.act);
  uint16_t *eout = (uint16_t *)at(o.eout);
  uint16_t *sparse = (uint16_t *)at(o.sparse);

  auto begin = [&](int i) {
    if (clock) clock->begin(i);
  };
  auto end = [&](int i) {
    if (clock) clock->end(i);
  };
  const bool has_shared = L.shared_intermediate > 0;
  uint16_t *shared_out = has_shared ? (uint16_t *)at(o.shared_out) : nullptr;
  uint16_t *z = has_shared ? (uint16_t *)at(o.z) : nullptr;
  const bool fuse_step = step && o.decode && (size_t)T * H * 2 <= (size_t)kDecodeStepLds && H % 8 == 0;
  if (step && !fuse_step) {
    // attention_residual and normalized_attention (decoder_layer_forward.rs:111-116)
    hipError_t e = launch_add_rms_norm(step->h, step->a, step->w, step->eps, T, H, step->r, step->n, s);
    if (e != hipSuccess) return hip_fail(kBlockOp, e);
  }
  auto finish = [&]() {  // attention_residual + mlp_output (decoder_layer_forward.rs:171-173)
    if (!step || fuse_step) return ok();
    hipError_t e = launch_add_bf16(step->r, y, (int64_t)T * H, step->out, s);
    return e == hipSuccess ? ok() : hip_fail(kBlockOp, e);
  };

  if (o.decode) {
    DecodeArgs d{};
    d.T = T;
    d.A = A;
    d.H = H;
    d.E = E;
    d.k = k;
    d.I = I;
    d.Is = has_shared ? L.shared_intermediate : 0;
    d.normalize = L.normalize_top_k;
    d.x = x;
    d.router_w = L.router_w;
    d.router_bias = L.router_bias;
    if (!L.router_w) {
      d.rq_w = L.router_q.w;
      d.rq_s = L.router_q.scales;
      d.rq_b = L.router_q.biases;
      d.rq_bits = L.router_q.bits;
      d.rq_group = L.router_q.group_size;
      d.rq_w_rs = words_per_row(L.router_q);
      d.rq_sb_rs = groups_per_row(L.router_q);
    }
    const astro_moe_affine &g = L.gate_up.w ? L.gate_up : L.gate;
    const astro_moe_affine &u = L.gate_up.w ? L.gate_up : L.up;
    const int64_t up_off = L.gate_up.w ? (int64_t)I : 0;
    d.gu_w_rs = words_per_row(g);
    d.gu_sb_rs = groups_per_row(g);
    d.gu_w_es = (int64_t)g.out_features * d.gu_w_rs;
    d.gu_sb_es = (int64_t)g.out_features * d.gu_sb_rs;
    d.gate_w = g.w;
    d.gate_s = g.scales;
    d.gate_b = g.biases;
    d.up_w = u.w + up_off * d.gu_w_rs;
    d.up_s = u.scales + up_off * d.gu_sb_rs;
    d.up_b = u.biases + up_off * d.gu_sb_rs;
    d.gu_bits = g.bits;
    d.gu_group = g.group_size;
    d.down_w = L.down.w;
    d.down_s = L.down.scales;
    d.down_b = L.down.biases;
    d.dn_w_rs = words_per_row(L.down);
    d.dn_sb_rs = groups_per_row(L.down);
    d.dn_w_es = (int64_t)H * d.dn_w_rs;
    d.dn_sb_es = (int64_t)H * d.dn_sb_rs;
    d.dn_bits = L.down.bits;
    d.dn_group = L.down.group_size;
    if (has_shared) {
      d.sg_w = L.shared_gate.w;
      d.sg_s = L.shared_gate.scales;
      d.sg_b = L.shared_gate.biases;
      d.su_w = L.shared_up.w;
      d.su_s = L.shared_up.scales;
      d.su_b = L.shared_up.biases;
      d.sg_w_rs = words_per_row(L.shared_gate);
      d.sg_sb_rs = groups_per_row(L.shared_gate);
      d.sg_bits = L.shared_gate.bits;
      d.sg_group = L.shared_gate.group_size;
      d.sd_w = L.shared_down.w;
      d.sd_s = L.shared_down.scales;
      d.sd_b = L.shared_down.biases;
      d.sd_w_rs = words_per_row(L.shared_down);
      d.sd_sb_rs = groups_per_row(L.shared_down);
      d.sd_bits = L.shared_down.bits;
      d.sd_group = L.shared_down.group_size;
      d.sz_w = L.shared_expert_gate.w;
      d.sz_s = L.shared_expert_gate.scales;
      d.sz_b = L.shared_expert_gate.biases;
      d.sz_bits = L.shared_expert_gate.bits;
      d.sz_group = L.shared_expert_gate.group_size;
    }
    d.logits = logits;
    d.scores = scores;
    d.idx = idx;
    d.sorted_order = sorted_order;
    d.inverse_order = inverse;
    d.sorted_ids = sorted_ids;
    d.offsets = offsets;
    uint32_t *groups = (uint32_t *)at(o.groups);
    d.n_groups = groups;
    d.g_expert = groups + 1;
    d.g_start = groups + 1 + 64;
    d.g_count = groups + 1 + 128;
    d.g_tokens = groups + 1 + 192;
    d.act = act;
    d.act_ld = o.act_ld;
    d.down_out = eout;
    d.z = z;
    d.sparse = sparse;
    d.y = y;
    d.router_blocks = (E + 3) / 4;
    d.shared_pair_blocks = has_shared ? (d.Is + 4 * kDecodeRowsPerWave - 1) / (4 * kDecodeRowsPerWave) : 0;
    d.max_groups = std::min(A, E);
    if (fuse_step) {
      d.h_in = step->h;
      d.a_in = step->a;
      d.norm_w = step->w;
      d.eps = step->eps;
      d.r_out = step->r;
      d.x_out = step->n;
      d.ffn_out = step->out;
    }
    d.unsorted = verification;
    // compact pages: sorted by slot over every slot id (run_sparse's bucket count)
    d.buckets = E;
    if (L.slot_of_expert) {
      d.slot_of_expert = L.slot_of_expert;
      d.slots = (uint32_t *)at(o.slots);
      d.missing = (uint32_t *)at(o.missing);
      d.slot_count = expert_capacity(L);
      d.buckets = std::max(E, d.slot_count);
    }
    if (!decode_supported(d)) return fail(ASTRO_MOE_UNSUPPORTED, kBlockOp, "decode path geometry");
    // kernel-attached events: router | gate/up (shared gate/up, routing, sort inside) |
    // down (shared down and the combine inside)
    hipEvent_t kev[8];
    if (clock) {
      // router | gate/up | down | routing (its own kernel from kDecodeRouteOnceT tokens)
      const int st[4] = {0, 3, 4, 1};
      const int nst = T >= kDecodeRouteOnceT ? 4 : 3;
      for (int i = 0; i < nst; ++i) {
        clock->used[st[i]] = true;
        kev[2 * i] = clock->ev[2 * st[i]];
        kev[2 * i + 1] = clock->ev[2 * st[i] + 1];
      }
    }
    hipError_t e = launch_decode_block(d, s, clock ? kev : nullptr);
    if (e != hipSuccess) return hip_fail(kBlockOp, e);
    return finish();
  }

  begin(0);
  hipError_t e = run_router(L, x, T, logits, s);
  end(0);
  begin(1);
  // the route kernel's wave per token also writes x's group sums and paired copy when the
  // sorted path's gate/up takes them (run_sparse's plan, which only reads the layer and the
  // layout) and the shared expert's output gate z (run_shared_gate's qgemv rows)
  RouteExtras ex;
  if (((uintptr_t)x & 15) == 0 && H % 32 == 0) {
    if (plan_sparse(L, x, T, k, o, ws, true).paired_x) {
      const astro_moe_affine &gu_w = L.gate_up.w ? L.gate_up : L.gate;
      ex.x = x;
      ex.H = H;
      ex.g = gu_w.group_size;
      ex.xsum = (float *)at(o.xsum_x);
      ex.paired = (uint16_t *)at(o.xpair);
    }
    const astro_moe_affine &zg = L.shared_expert_gate;
    if (has_shared && (zg.bits == 4 || zg.bits == 8) && zg.group_size % 32 == 0) {
      ex.x = x;
      ex.H = H;
      ex.zw = zg.w;
      ex.zs = zg.scales;
      ex.zb = zg.biases;
      ex.zbits = zg.bits;
      ex.zgroup = zg.group_size;
      ex.z = z;
    }
  }
  if (e == hipSuccess) e = launch_route_topk(logits, T, E, k, L.normalize_top_k, idx, scores, s, ex);
  // compact pages (forward_moe_paged, paged_execution.rs:98-139): the expert ids become page
  // slots (qwen3_5_moe_remap_expert_page_slots, split_page_route.rs:79-105) before the sort
  const uint32_t *ids = idx;
  if (e == hipSuccess && L.slot_of_expert) {
    uint32_t *slots = (uint32_t *)at(o.slots), *missing = (uint32_t *)at(o.missing);
    e = launch_zero_u32(missing, 1, s);
    if (e == hipSuccess) e = launch_remap_slots(idx, A, L.slot_of_expert, E, slots, missing, s);
    ids = slots;
  }
  end(1);
  if (e != hipSuccess) return hip_fail(kBlockOp, e);
  // a verification window keeps the unsorted reduction at every length
  // (forward_moe_resident_target_verification, resident_execution.rs:146-208)
  e = run_sparse(L, x, T, k, ids, scores, o, ws, true, y, s, clock, verification, ex.xsum != nullptr,
                 ex.z != nullptr);
  if (e != hipSuccess) return hip_fail(kBlockOp, e);
  return finish();
}

}  // namespace

extern "C" {

int astro_moe_abi_version(void) { return ASTRO_MOE_ABI_VERSION; }

int astro_moe_workspace_bytes(const astro_moe_layer *layer, int32_t tokens, size_t *bytes) {
  int rc = check_layer(kBlockOp, layer);
  if (rc) return rc;
  if (tokens < 0 || !bytes) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "token count must not be negative");
  *bytes = block_layout(*layer, tokens, layer->top_k, true).total;
  return ok();
}

int astro_moe_workspace_layout(const astro_moe_layer *layer, int32_t tokens,
                               astro_moe_workspace_view *view) {
  int rc = check_layer(kBlockOp, layer);
  if (rc) return rc;
  if (tokens < 0 || !view) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "token count must not be negative");
  const Layout o = block_layout(*layer, tokens, layer->top_k, true);
  view->total_bytes = o.total;
  view->sorted_path = (int64_t)tokens * layer->top_k >= 64;
  view->logits = o.logits;
  view->indices = o.idx;
  view->scores = o.scores;
  view->sorted_order = o.sorted_order;
  view->inverse_order = o.inverse;
  view->sorted_ids = o.sorted_ids;
  view->expert_offsets = o.offsets;
  view->activated = o.act;
  view->activated_ld = (size_t)o.act_ld;
  view->expert_out = o.eout;
  view->sparse = o.sparse;
  view->shared_out = o.shared_out;
  view->shared_gate_logits = o.z;
  view->expert_slots = o.slots;
  view->missing_slots = o.missing;
  view->tile_expert = o.decode ? 0 : o.tile_expert;
  view->tile_row0 = o.decode ? 0 : o.tile_row0;
  view->tile_count = o.decode ? 0 : o.tile_count;
  view->max_tiles = o.decode ? 0 : (size_t)o.max_tiles;
  view->activated_paired = !o.decode && view->sorted_path &&
                           plan_sparse(*layer, nullptr, tokens, layer->top_k, o, nullptr, true).act_paired;
  return ok();
}

int astro_moe_block_forward(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                            uint16_t *y, void *workspace, size_t workspace_bytes, void *stream) {
  return run_block(layer, x, tokens, y, workspace, workspace_bytes, stream, nullptr);
}

}  // extern "C"

// The no-allocation entry point's workspace: one static device array per GPU (each device
// holds its own copy at its own address).  In host code `scratch` names a host-side stand-in,
// not device memory: only the address hipGetSymbolAddress returns for the current device is
// ever passed to a kernel.
static __device__ __align__(256) char scratch[ASTRO_MOE_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];  // per device, looked up on its first call

int device_scratch(const char *op, void **ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(op, e);
  if (dev < 0 || dev >= kMaxDevices) return fail(ASTRO_MOE_UNSUPPORTED, op, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(op, e);
    if (!p) return fail(ASTRO_MOE_HIP_ERROR, op, "the static scratch array has no device address");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return ASTRO_MOE_OK;
}

}  // namespace

extern "C" {

int astro_moe_block_forward_no_alloc(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                                     uint16_t *y, void *stream) {
  size_t need = 0;
  int rc = astro_moe_workspace_bytes(layer, tokens, &need);
  if (rc) return rc;
  if (need > ASTRO_MOE_STATIC_SCRATCH_BYTES)
    return fail(ASTRO_MOE_WORKSPACE_TOO_SMALL, kBlockOp,
                "the no-allocation entry point's static scratch is too small for %d tokens: "
                "ASTRONOMICAL_MLX_ACTIVE_MEMORY_LIMIT_EXCEEDED active_bytes=0 allocation_bytes=%zu "
                "allowed_bytes=%zu",
                (int)tokens, need, (size_t)ASTRO_MOE_STATIC_SCRATCH_BYTES);
  if (tokens == 0) return ok();
  void *ws = nullptr;
  rc = device_scratch(kBlockOp, &ws);
  if (rc) return rc;
  return run_block(layer, x, tokens, y, ws, ASTRO_MOE_STATIC_SCRATCH_BYTES, stream, nullptr);
}

// forward_moe_resident_target_verification (resident_execution.rs:146-208): the rows of an MTP
// verification window stay unsorted, so each output row equals the one-token block of its row
// (the rollback boundary after a rejected draft).  The window runs in pieces the decode kernels
// take whole (at most 8 tokens and 64 assignments, unsorted combine), or one token at a time
// when they do not apply.
int astro_moe_block_forward_verification(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                                         uint16_t *y, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_layer(kBlockOp, layer);
  if (rc) return rc;
  if (tokens < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "token count must not be negative");
  if (tokens == 0) return ok();
  if (!x || !y) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "hidden states and output must be non-null");
  const astro_moe_layer &L = *layer;
  int piece = std::max(1, std::min({8, 64 / std::max(1, L.top_k), (int)tokens}));
  if (!decode_path(L, piece)) piece = 1;
  const int64_t H = L.hidden;
  for (int32_t t0 = 0; t0 < tokens; t0 += piece) {
    const int32_t n = std::min<int32_t>(piece, tokens - t0);
    rc = run_block(layer, x + t0 * H, n, y + t0 * H, workspace, workspace_bytes, stream, nullptr, nullptr, true);
    if (rc) return rc;
  }
  return ok();
}

int astro_moe_verification_workspace_bytes(const astro_moe_layer *layer, int32_t tokens, size_t *bytes) {
  int rc = check_layer(kBlockOp, layer);
  if (rc) return rc;
  if (tokens < 0 || !bytes) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "token count and output must be valid");
  const astro_moe_layer &L = *layer;
  int piece = std::max(1, std::min({8, 64 / std::max(1, L.top_k), (int)std::max(tokens, 1)}));
  if (!decode_path(L, piece)) piece = 1;
  *bytes = block_layout(L, piece, L.top_k, true).total;
  return ok();
}

int astro_moe_block_forward_attributed(const astro_moe_layer *layer, const uint16_t *x,
                                       int32_t tokens, uint16_t *y, void *workspace,
                                       size_t workspace_bytes, void *stream, float *stage_ms) {
  if (!stage_ms) return fail(ASTRO_MOE_INVALID_ARGUMENT, kBlockOp, "stage time output must be non-null");
  hipEvent_t ev[2 * ASTRO_MOE_STAGES];
  for (int i = 0; i < 2 * ASTRO_MOE_STAGES; ++i) {
    hipError_t e = hipEventCreate(&ev[i]);
    if (e != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      return hip_fail(kBlockOp, e);
    }
  }
  StageClock clock{ev, (hipStream_t)stream, {}};
  int rc = run_block(layer, x, tokens, y, workspace, workspace_bytes, stream, &clock);
  hipError_t e = rc == ASTRO_MOE_OK ? hipStreamSynchronize((hipStream_t)stream) : hipSuccess;
  for (int i = 0; i < ASTRO_MOE_STAGES && rc == ASTRO_MOE_OK && e == hipSuccess; ++i) {
    stage_ms[i] = 0.0f;
    if (clock.used[i]) e = hipEventElapsedTime(&stage_ms[i], ev[2 * i], ev[2 * i + 1]);
  }
  if (rc == ASTRO_MOE_OK && e != hipSuccess) rc = hip_fail(kBlockOp, e);
  for (int i = 0; i < 2 * ASTRO_MOE_STAGES; ++i) (void)hipEventDestroy(ev[i]);
  return rc == ASTRO_MOE_OK ? ok() : rc;
}

int astro_moe_router_logits(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                            uint16_t *logits, void *stream) {
  int rc = check_layer(kRouteOp, layer);
  if (rc) return rc;
  if (tokens < 0 || (tokens > 0 && (!x || !logits)))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kRouteOp, "router inputs must be non-null");
  if (tokens == 0) return ok();
  hipError_t e = run_router(*layer, x, tokens, logits, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(kRouteOp, e);
}

int astro_moe_route_topk(const uint16_t *logits, int32_t tokens, int32_t experts, int32_t top_k,
                         int32_t normalize, uint32_t *indices, uint16_t *scores, void *stream) {
  // validate_router_arguments (routing.rs:123-153)
  if (tokens < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, kRouteOp, "router logits must include token and expert dimensions");
  if (experts <= 0 || top_k <= 0 || top_k > experts)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kRouteOp,
                "selected expert count must be positive and no larger than the router dimension");
  if (experts > 1024 || top_k > 64)
    return fail(ASTRO_MOE_UNSUPPORTED, kRouteOp, "the router kernel supports at most 1024 experts and top-64");
  if (tokens == 0) return ok();
  if (!logits || !indices || !scores) return fail(ASTRO_MOE_INVALID_ARGUMENT, kRouteOp, "router buffers must be non-null");
  hipError_t e = launch_route_topk(logits, tokens, experts, top_k, normalize, indices, scores,
                                   (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(kRouteOp, e);
}

static size_t sort_ws_bytes(int A, int E) {
  const int mt = sort_max_tiles(A, E);
  return align_up(((size_t)E + 2) * 4) + 2 * align_up((size_t)mt * 4) + align_up(4) +
         align_up(sort_scratch_bytes(A, E));
}

int astro_moe_sort_workspace_bytes(int32_t assignments, int32_t experts, size_t *bytes) {
  if (assignments < 0 || experts <= 0 || !bytes)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kSortOp, "expert assignments and expanded hidden states have invalid shapes");
  if (experts > 1024) return fail(ASTRO_MOE_UNSUPPORTED, kSortOp, "the sort kernels support at most 1024 experts");
  *bytes = sort_ws_bytes(assignments, experts);
  return ok();
}

int astro_moe_sort_assignments(const uint32_t *ids, int32_t assignments, int32_t experts,
                               uint32_t *sorted_order, uint32_t *inverse_order,
                               uint32_t *sorted_ids, uint32_t *expert_offsets, void *workspace,
                               size_t workspace_bytes, void *stream) {
  if (assignments < 0 || experts <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kSortOp, "expert assignments and expanded hidden states have invalid shapes");
  if (experts > 1024) return fail(ASTRO_MOE_UNSUPPORTED, kSortOp, "the sort kernels support at most 1024 experts");
  const size_t need = sort_ws_bytes(assignments, experts);
  if (!workspace || workspace_bytes < need) return workspace_fail(kSortOp, need, workspace ? workspace_bytes : 0);
  if (assignments > 0 && (!ids || !sorted_order || !inverse_order || !sorted_ids))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kSortOp, "assignment buffers must be non-null");
  hipStream_t s = (hipStream_t)stream;
  char *ws = (char *)workspace;
  const int mt = sort_max_tiles(assignments, experts);
  uint32_t *off = (uint32_t *)ws;
  uint32_t *te = (uint32_t *)(ws + align_up(((size_t)experts + 2) * 4));
  uint32_t *tr = (uint32_t *)((char *)te + align_up((size_t)mt * 4));
  uint32_t *tc = (uint32_t *)((char *)tr + align_up((size_t)mt * 4));
  uint32_t *scr = (uint32_t *)((char *)tc + align_up(4));
  hipError_t e = launch_sort(ids, assignments, experts, sorted_order, inverse_order, sorted_ids,
                             off, te, tr, tc, scr, s);
  if (e == hipSuccess && expert_offsets)
    e = hipMemcpyAsync(expert_offsets, off, ((size_t)experts + 1) * 4, hipMemcpyDeviceToDevice, s);
  return e == hipSuccess ? ok() : hip_fail(kSortOp, e);
}

int astro_moe_invert_assignment_order(const uint32_t *sorted_order, int32_t n,
                                      uint32_t *inverse_order) {
  if (n < 0 || (n > 0 && (!sorted_order || !inverse_order)))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kPermOp, "assignment permutation length exceeds u32");
  std::vector<uint8_t> seen((size_t)n, 0);
  for (int32_t s = 0; s < n; ++s) {
    const uint32_t o = sorted_order[s];
    if (o >= (uint32_t)n)
      return fail(ASTRO_MOE_INVALID_ARGUMENT, kPermOp, "assignment permutation contains an out-of-range slot");
    if (seen[o]) return fail(ASTRO_MOE_INVALID_ARGUMENT, kPermOp, "assignment permutation contains a duplicate slot");
    seen[o] = 1;
    inverse_order[o] = (uint32_t)s;
  }
  for (int32_t s = 0; s < n; ++s)
    if (!seen[s]) return fail(ASTRO_MOE_INVALID_ARGUMENT, kPermOp, "assignment permutation is missing a slot");
  return ok();
}

int astro_moe_gather_qmm_workspace_bytes(int32_t rows, int32_t experts, size_t *bytes) {
  if (rows < 0 || experts <= 0 || !bytes)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kGatherOp, "gather_qmm requires at least one index array");
  *bytes = 3 * align_up((size_t)rows * 4) + sort_ws_bytes(rows, experts);
  return ok();
}

int astro_moe_gather_qmm(const uint16_t *x, const uint32_t *x_rows, int32_t rows,
                         const astro_moe_affine *w, const uint32_t *ids, int32_t sorted_indices,
                         uint16_t *out, void *workspace, size_t workspace_bytes, void *stream) {
  (void)sorted_indices;  // a promise about id order; kernel selection here ignores it
  int rc = check_affine(kGatherOp, w, -1);
  if (rc) return rc;
  if (rows < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, kGatherOp, "activation and weight arrays must both have rank at least two");
  if (rows == 0) return ok();
  if (!x || !ids || !out) return fail(ASTRO_MOE_INVALID_ARGUMENT, kGatherOp, "gather_qmm requires at least one index array");
  size_t need = 0;
  astro_moe_gather_qmm_workspace_bytes(rows, w->experts, &need);
  if (!workspace || workspace_bytes < need) return workspace_fail(kGatherOp, need, workspace ? workspace_bytes : 0);
  hipStream_t s = (hipStream_t)stream;
  char *ws = (char *)workspace;
  const size_t ra = align_up((size_t)rows * 4);
  uint32_t *so = (uint32_t *)ws, *inv = (uint32_t *)(ws + ra), *sid = (uint32_t *)(ws + 2 * ra);
  char *sw = ws + 3 * ra;
  const int E = w->experts, mt = sort_max_tiles(rows, E);
  uint32_t *off = (uint32_t *)sw;
  uint32_t *te = (uint32_t *)(sw + align_up(((size_t)E + 2) * 4));
  uint32_t *tr = (uint32_t *)((char *)te + align_up((size_t)mt * 4));
  uint32_t *tc = (uint32_t *)((char *)tr + align_up((size_t)mt * 4));
  uint32_t *scr = (uint32_t *)((char *)tc + align_up(4));
  hipError_t e = launch_sort(ids, rows, E, so, inv, sid, off, te, tr, tc, scr, s);
  if (e != hipSuccess) return hip_fail(kGatherOp, e);
  GemmArgs g{};
  g.A = x;
  g.lda = w->in_features;
  g.a_rows = so;
  g.a_div = 1;
  g.a_rows2 = x_rows;
  g.K = w->in_features;
  g.N = w->out_features;
  set_weights(g, *w, nullptr, 0);
  g.tile_expert = te;
  g.tile_row0 = tr;
  g.tile_count = tc;
  g.expert_offsets = off;
  g.max_tiles = mt;
  g.C = out;
  g.ldc = w->out_features;
  g.c_rows = so;
  e = launch_grouped_gemm(g, kEpiPlain, s);
  return e == hipSuccess ? ok() : hip_fail(kGatherOp, e);
}

int astro_moe_quantized_matmul(const uint16_t *x, int32_t rows, const astro_moe_affine *w,
                               uint16_t *out, void *stream) {
  int rc = check_affine(kQmmOp, w, -1);
  if (rc) return rc;
  if (w->experts != 1) return fail(ASTRO_MOE_INVALID_ARGUMENT, kQmmOp, "a plain quantized matmul takes one weight matrix");
  if (rows < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, kQmmOp, "activation and weight arrays must both have rank at least two");
  if (rows == 0) return ok();
  if (!x || !out) return fail(ASTRO_MOE_INVALID_ARGUMENT, kQmmOp, "quantized matmul buffers must be non-null");
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (rows <= kVerifyRows && verify_qmv_supported(w->in_features, w->bits, w->group_size, x, w->w)) {
    // a few rows: the multi-token QMV (each row's bits are those of a one-row call)
    e = launch_verify_qmv(x, rows, w->in_features, w->w, w->scales, w->biases, w->out_features, w->bits,
                          w->group_size, false, out, s);
  } else if (w->out_features < 16) {
    e = launch_qgemv_rows(x, rows, w->in_features, w->w, w->scales, w->biases, w->out_features,
                          w->bits, w->group_size, out, s);
  } else {
    GemmArgs g{};
    g.A = x;
    g.lda = w->in_features;
    g.a_div = 1;
    g.K = w->in_features;
    g.N = w->out_features;
    g.M = rows;
    set_weights(g, *w, nullptr, 0);
    g.C = out;
    g.ldc = w->out_features;
    e = launch_grouped_gemm(g, kEpiPlain, s);
  }
  return e == hipSuccess ? ok() : hip_fail(kQmmOp, e);
}

// qwen3_5_target_verification_quantized_linear (target_verification_quantized_linear.rs:232-330)
// with the checks of validate_target_verification_projection (:378-447).  One kernel serves
// both of the reference's dispatch arms: its outputs are token-local by construction.
int astro_moe_verification_quantized_linear(const void *activations, int32_t batch, int32_t tokens,
                                            int32_t in_features, const astro_moe_affine *w, int32_t dtype,
                                            void *out, void *stream) {
  const char *op = "project Qwen3.5 target-verification tokens";
  if (batch <= 0 || tokens <= 0 || in_features <= 0 || !w || w->experts != 1 || w->out_features <= 0 ||
      w->in_features <= 0 || ((int64_t)w->in_features * w->bits) / 32 <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "target-verification arrays must have positive rank-three activations and rank-two weights");
  if ((w->group_size != 32 && w->group_size != 64 && w->group_size != 128) ||
      (w->bits != 2 && w->bits != 3 && w->bits != 4 && w->bits != 5 && w->bits != 6 && w->bits != 8))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "target-verification affine metadata is not supported by MLX");
  if (((int64_t)w->in_features * w->bits) % 32 != 0 || w->in_features != in_features ||
      in_features % w->group_size != 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "target-verification affine arrays do not match activation and weight geometry");
  if (!activations || !out || !w->w || !w->scales || !w->biases)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "target-verification buffers must be non-null");
  if (dtype != ASTRO_MOE_DTYPE_BF16 && dtype != ASTRO_MOE_DTYPE_F16)
    return fail(ASTRO_MOE_UNSUPPORTED, op,
                "the verification kernel reads bfloat16 or float16 activations, scales and biases");
  if ((int64_t)batch * tokens > (int64_t)INT32_MAX / in_features)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "target-verification activations are too large");
  if (!verify_qmv_supported(in_features, w->bits, w->group_size, activations, w->w))
    return fail(ASTRO_MOE_UNSUPPORTED, op,
                "the verification kernel needs 4-, 5- or 8-bit codes, an input width that is a multiple of "
                "128 and 16-byte aligned activations and codes");
  const hipError_t e =
      launch_verify_qmv((const uint16_t *)activations, batch * tokens, in_features, w->w, w->scales, w->biases,
                        w->out_features, w->bits, w->group_size, dtype == ASTRO_MOE_DTYPE_F16, (uint16_t *)out,
                        (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(op, e);
}

int astro_moe_swiglu(const uint16_t *gate, const uint16_t *up, int64_t n, uint16_t *out,
                     void *stream) {
  if (n < 0 || (n > 0 && (!gate || !up || !out)))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, "apply a compiled MLX SwiGLU graph", "SwiGLU buffers must be non-null");
  hipError_t e = launch_swiglu(gate, up, n, out, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail("apply a compiled MLX SwiGLU graph", e);
}

int astro_moe_sorted_weighted_sum(const uint16_t *sorted_outputs, const uint32_t *inverse_order,
                                  const uint16_t *scores, int32_t tokens, int32_t top_k,
                                  int32_t dim, uint16_t *out, void *stream) {
  // sorted_expert_weighted_sum_inner (weighted_sum.rs:129-156)
  if (tokens < 0 || top_k < 0 || dim <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kReduceOp,
                "sorted expert outputs, inverse order, and scores have invalid shapes or dtypes");
  if (tokens == 0) return ok();
  if (!out || (top_k > 0 && (!sorted_outputs || !inverse_order || !scores)))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kReduceOp, "sorted expert outputs and inverse order must match selected scores");
  hipError_t e = launch_combine(sorted_outputs, inverse_order, scores, tokens, top_k, dim, 1,
                                nullptr, nullptr, nullptr, out, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(kReduceOp, e);
}

int astro_moe_unsorted_weighted_sum(const uint16_t *outputs, const uint16_t *scores,
                                    int32_t tokens, int32_t top_k, int32_t dim, uint16_t *out,
                                    void *stream) {
  if (tokens < 0 || top_k < 0 || dim <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kReduceOp, "unsorted expert outputs and scores must include an assignment axis");
  if (tokens == 0) return ok();
  if (!out || (top_k > 0 && (!outputs || !scores)))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kReduceOp, "unsorted expert outputs and scores must be non-null");
  hipError_t e = launch_combine(outputs, nullptr, scores, tokens, top_k, dim, 0, nullptr, nullptr,
                                nullptr, out, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(kReduceOp, e);
}

int astro_moe_combine_shared(const uint16_t *sparse, const uint16_t *shared_out,
                             const uint16_t *gate_logits, int32_t tokens, int32_t dim,
                             uint16_t *out, void *stream) {
  if (tokens < 0 || dim <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kCombineOp, "shared expert output must match the combined sparse-expert shape");
  if (tokens == 0) return ok();
  if (!sparse || !shared_out || !gate_logits || !out)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kCombineOp, "shared expert gate must provide one logit per token");
  hipError_t e = launch_combine_shared(sparse, shared_out, gate_logits, tokens, dim, out, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(kCombineOp, e);
}

int astro_moe_shared_expert_workspace_bytes(const astro_moe_layer *layer, int32_t tokens,
                                            size_t *bytes) {
  if (!layer || tokens < 0 || !bytes || layer->shared_intermediate <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kCombineOp, "the layer has no shared expert");
  *bytes = align_up((size_t)tokens * layer->shared_intermediate * 2);
  return ok();
}

int astro_moe_shared_expert(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                            uint16_t *shared_out, uint16_t *gate_logits, void *workspace,
                            size_t workspace_bytes, void *stream) {
  int rc = check_layer(kCombineOp, layer);
  if (rc) return rc;
  if (layer->shared_intermediate <= 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, kCombineOp, "the layer has no shared expert");
  if (tokens < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, kCombineOp, "token count must not be negative");
  if (tokens == 0) return ok();
  const size_t need = align_up((size_t)tokens * layer->shared_intermediate * 2);
  if (!workspace || workspace_bytes < need) return workspace_fail(kCombineOp, need, workspace ? workspace_bytes : 0);
  if (!x || !shared_out || !gate_logits) return fail(ASTRO_MOE_INVALID_ARGUMENT, kCombineOp, "shared expert buffers must be non-null");
  hipError_t e = run_shared(*layer, x, tokens, (uint16_t *)workspace, shared_out, gate_logits,
                            (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(kCombineOp, e);
}


int astro_moe_remap_expert_slots(const uint32_t *expert_ids, int32_t n, const uint32_t *slot_of_expert,
                                 int32_t experts, uint32_t *slots, uint32_t *missing_count, void *stream) {
  const char *op = "remap Qwen3.5-MoE expert page slots";
  if (n < 0 || experts <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "assignment count must not be negative and the expert capacity positive");
  if (n == 0) return ok();
  if (!expert_ids || !slot_of_expert || !slots)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "expert ids, the slot map and the slot output must be non-null");
  hipError_t e = launch_remap_slots(expert_ids, n, slot_of_expert, experts, slots, missing_count, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(op, e);
}

int astro_moe_gather_assignments(const uint32_t *ids, const uint16_t *scores, const uint32_t *positions,
                                 int32_t n, uint32_t *out_ids, uint16_t *out_scores, void *stream) {
  const char *op = "build Qwen3.5-MoE split expert page route";
  if (n < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "assignment count must not be negative");
  if (n == 0) return ok();
  if (!positions || (out_ids && !ids) || (out_scores && !scores))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "positions and the source of every requested output must be non-null");
  hipError_t e = launch_gather_assignments(ids, scores, positions, n, out_ids, out_scores, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(op, e);
}

static int check_page(const char *op, const astro_moe_layer *page) {
  if (!page) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "page description must be non-null");
  if (page->hidden <= 0 || page->intermediate <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "hidden and intermediate sizes must be positive");
  return check_routed(op, page, expert_capacity(*page));
}

static const char *const kStreamedOp = "run Qwen3.5-MoE experts from a streamed page";

int astro_moe_streamed_sparse_workspace_bytes(const astro_moe_layer *page, int32_t tokens, int32_t per_token,
                                              size_t *bytes) {
  int rc = check_page(kStreamedOp, page);
  if (rc) return rc;
  if (tokens < 0 || per_token <= 0 || !bytes)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kStreamedOp, "token count must not be negative and assignments per token positive");
  *bytes = block_layout(*page, tokens, per_token, false).total;
  return ok();
}

int astro_moe_streamed_sparse_forward(const astro_moe_layer *page, const uint16_t *x, int32_t tokens,
                                      const uint32_t *slots, const uint16_t *scores, int32_t per_token,
                                      uint16_t *sparse, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_page(kStreamedOp, page);
  if (rc) return rc;
  if (tokens < 0 || per_token <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kStreamedOp, "token count must not be negative and assignments per token positive");
  if (tokens == 0) return ok();
  if (!x || !slots || !scores || !sparse)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, kStreamedOp, "hidden states, slots, scores and output must be non-null");
  const Layout o = block_layout(*page, tokens, per_token, false);
  if (!workspace || workspace_bytes < o.total)
    return workspace_fail(kStreamedOp, o.total, workspace ? workspace_bytes : 0);
  hipError_t e = run_sparse(*page, x, tokens, per_token, slots, scores, o, (char *)workspace, false, sparse,
                            (hipStream_t)stream, nullptr);
  return e == hipSuccess ? ok() : hip_fail(kStreamedOp, e);
}

int astro_moe_add(const uint16_t *a, const uint16_t *b, int64_t n, uint16_t *out, void *stream) {
  const char *op = "add";
  if (n < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "element count must not be negative");
  if (n == 0) return ok();
  if (!a || !b || !out) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "operands and output must be non-null");
  hipError_t e = launch_add_bf16(a, b, n, out, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(op, e);
}

int astro_moe_selftest_bf16_rounding(uint64_t *mismatches, void *stream) {
  const char *op = "self-test the bf16 rounding";
  if (!mismatches) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "the mismatch counter must be non-null");
  hipError_t e = launch_selftest_bf16((unsigned long long *)mismatches, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(op, e);
}

// ------------------------------------------------------------------ the decoder step around the block

int astro_moe_add_rms_norm(const uint16_t *hidden, const uint16_t *attention_out, const uint16_t *norm_weight,
                           float eps, int32_t tokens, int32_t hidden_size, uint16_t *residual_out,
                           uint16_t *normed_out, void *stream) {
  const char *op = "apply MLX RMS normalization";  // mlx_operations.rs:97
  if (tokens < 0 || hidden_size <= 0)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "token count must not be negative and the hidden size positive");
  if (hidden_size > 8192 || hidden_size % 8 != 0)
    return fail(ASTRO_MOE_UNSUPPORTED, op, "the normalization kernel supports hidden sizes that are multiples of 8 up to 8192");
  if (!(eps >= 0.0f)) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "epsilon must be a non-negative number");
  if (tokens == 0) return ok();
  if (!hidden || !norm_weight || !normed_out)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "hidden states, weight and output must be non-null");
  hipError_t e = launch_add_rms_norm(hidden, attention_out, norm_weight, eps, tokens, hidden_size,
                                     residual_out, normed_out, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(op, e);
}

static size_t ffn_extra_bytes(int T, int H) { return 3 * align_up((size_t)T * H * 2); }

int astro_moe_decoder_ffn_workspace_bytes(const astro_moe_layer *layer, int32_t tokens, size_t *bytes) {
  size_t blk = 0;
  int rc = astro_moe_workspace_bytes(layer, tokens, &blk);
  if (rc) return rc;
  *bytes = align_up(blk) + ffn_extra_bytes(tokens, layer->hidden);
  return ok();
}

int astro_moe_decoder_ffn_forward(const astro_moe_layer *layer, const uint16_t *hidden,
                                  const uint16_t *attention_out, const uint16_t *norm_weight, float eps,
                                  int32_t tokens, uint16_t *out, uint16_t *residual_out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  const char *op = "run the Qwen3.5 decoder feed-forward step";
  size_t blk = 0;
  int rc = astro_moe_workspace_bytes(layer, tokens, &blk);
  if (rc) return rc;
  const int H = layer->hidden;
  const size_t need = align_up(blk) + ffn_extra_bytes(tokens, H);
  if (!workspace || workspace_bytes < need) return workspace_fail(op, need, workspace ? workspace_bytes : 0);
  if (tokens == 0) return ok();
  if (!hidden || !norm_weight || !out) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "hidden states, weight and output must be non-null");
  if (!(eps >= 0.0f)) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "epsilon must be a non-negative number");
  if (H > 8192) return fail(ASTRO_MOE_UNSUPPORTED, op, "the normalization kernel supports hidden sizes up to 8192");
  // The router kernel of the fused decode step writes r while other workgroups still read the
  // hidden states and the attention output to form r themselves, so r may not share memory
  // with either input (an in-place residual update would feed r + a back into them).
  const size_t rows_bytes = (size_t)tokens * H * 2;
  auto overlaps = [&](const void *a, const void *b) {
    const char *pa = (const char *)a, *pb = (const char *)b;
    return a && b && pa < pb + rows_bytes && pb < pa + rows_bytes;
  };
  if (overlaps(residual_out, hidden) || overlaps(residual_out, attention_out))
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "residual output must not overlap the hidden states or the attention output");
  char *ws = (char *)workspace;
  uint16_t *r = (uint16_t *)(ws + align_up(blk));
  uint16_t *n = (uint16_t *)((char *)r + align_up((size_t)tokens * H * 2));
  uint16_t *y = (uint16_t *)((char *)n + align_up((size_t)tokens * H * 2));
  if (residual_out) r = residual_out;
  const DecoderStep step{hidden, attention_out, norm_weight, eps, r, n, out};
  return run_block(layer, n, tokens, y, workspace, blk, stream, nullptr, &step);
}

// route_laguna_experts (laguna/moe/router.rs:29-94) with the CPU selection order
int astro_moe_route_laguna(const uint16_t *logits, int32_t tokens, int32_t experts, int32_t top_k,
                           const float *correction_bias, double softcap, int32_t normalize,
                           uint32_t *indices, float *scores, void *stream) {
  const char *op = "route Laguna sparse experts";
  if (tokens < 0) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "router logits must include token and expert dimensions");
  if (experts <= 0 || top_k <= 0 || top_k > experts)
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op,
                "selected expert count must be positive and no larger than the router dimension");
  if (!(softcap >= 0.0))  // router_selection.rs:125-139
    return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "Laguna router logits, top-K, and softcap must describe a valid selection");
  if (experts > 1024 || top_k > 64)
    return fail(ASTRO_MOE_UNSUPPORTED, op, "the router kernel supports at most 1024 experts and top-64");
  if (tokens == 0) return ok();
  if (!logits || !indices || !scores) return fail(ASTRO_MOE_INVALID_ARGUMENT, op, "router buffers must be non-null");
  hipError_t e = launch_route_laguna(logits, tokens, experts, top_k, correction_bias, (float)softcap, normalize,
                                     indices, scores, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(op, e);
}

}  // extern "C"
