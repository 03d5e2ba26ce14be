// Decode path of the block (T <= 8 tokens, T*k <= 64 assignments): wavefront GEMVs
// instead of MFMA tiles, three kernels per layer:
//   D1  router GEMV (one wave per expert row);
//   D2  the shared expert's gate/up + SwiGLU and its output gate (no routing needed), and
//       routing (softmax/top-k, the sort of the assignments, the distinct-expert table),
//       recomputed by every routed workgroup, then the routed gate/up GEMV + SwiGLU: one
//       wave per (gate row, up row) pair of one selected expert, every token routed to it;
//   D3  per token: down GEMV rows of its k experts and of the shared expert (16 lanes per
//       row, the participants spread over 3 to 9 waves), then the weighted combine and the
//       shared expert's gated add.
// Affine rows are read once per distinct expert with 16 B per lane loads.  4-bit codes are
// turned into bf16 pairs (128 + q) with one and/or per pair and multiplied by
// v_dot2_f32_bf16; the per-group affine terms are applied per 32-input chunk:
//   sum_j x_j (s q_j + b) = s * sum_j (128 + q_j) x_j + (b - 128 s) * sum_j x_j.
//
// This header holds the device code and the launch templates of the decode path; the gate/up
// kernels (the bulk of the instantiations) are compiled in decode_gate_up.hip, one object per
// (code width, token count), and the rest in decode.hip.
#pragma once
#include "common.h"
#include "kernels.h"
#include "route_dev.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <type_traits>

namespace astro {

namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// (gate row, up row) pairs per wave in the gate/up GEMVs: one keeps each wave's serial
// instruction chain short; the chip has wave slots to spare at decode sizes
constexpr int kRowsPerWave = kDecodeRowsPerWave;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b),
                                         c, false);
}

__device__ __forceinline__ uint32_t pack_bf2_hw(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// 32 consecutive activations of one token, ready for the code dot products.  For 4-bit
// codes the bf16 pairs are (x0,x4),(x1,x5),(x2,x6),(x3,x7) per 8 inputs, matching the
// nibble pairs produced by (word >> 4m) & 0x000f000f; 8-bit codes use natural pairs.
struct XChunk {
  uint32_t p[16];
  float sum;
};

struct XRaw {
  u32x4 v[4];
};

__device__ __forceinline__ void load_xraw(XRaw &xr, const uint16_t *src) {
  const u32x4 *q = (const u32x4 *)src;
#pragma unroll
  for (int i = 0; i < 4; ++i) xr.v[i] = q[i];
}

template <int BITS>
__device__ __forceinline__ void convert_xchunk(XChunk &xc, const XRaw &xr) {
  uint32_t r[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[4 * i] = xr.v[i][0];
    r[4 * i + 1] = xr.v[i][1];
    r[4 * i + 2] = xr.v[i][2];
    r[4 * i + 3] = xr.v[i][3];
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s = dot2(r[j], 0x3f803f80u, s);
  xc.sum = s;
  if (BITS == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = r[4 * i], b = r[4 * i + 1], c = r[4 * i + 2], d = r[4 * i + 3];
      xc.p[4 * i + 0] = (a & 0xffffu) | (c << 16);
      xc.p[4 * i + 1] = (a >> 16) | (c & 0xffff0000u);
      xc.p[4 * i + 2] = (b & 0xffffu) | (d << 16);
      xc.p[4 * i + 3] = (b >> 16) | (d & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) xc.p[j] = r[j];
  }
}

template <int BITS>
__device__ __forceinline__ void load_xchunk(XChunk &xc, const uint16_t *src) {
  XRaw xr;
  load_xraw(xr, src);
  convert_xchunk<BITS>(xc, xr);
}

// codes of one 32-input chunk of one weight row: 4 words (4-bit) or 8 words (8-bit)
struct WChunk {
  u32x4 q[2];
  float s, b;
};

template <int BITS>
__device__ __forceinline__ void load_wchunk(WChunk &w, const uint32_t *row, const uint16_t *srow,
                                            const uint16_t *brow, int chunk, int group) {
  const u32x4 *p = (const u32x4 *)(row + chunk * BITS);
  w.q[0] = p[0];
  if (BITS == 8) w.q[1] = p[1];
  const int g = (chunk * 32) / group;
  w.s = bf2f(srow[g]);
  w.b = bf2f(brow[g]);
}

// sum over the chunk of x * (s*q + b)
template <int BITS>
__device__ __forceinline__ float chunk_dot(const WChunk &w, const XChunk &x) {
  float acc = 0.0f;
  if (BITS == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t word = w.q[0][i];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        acc = dot2(((word >> (4 * m)) & 0x000f000fu) | 0x43004300u, x.p[4 * i + m], acc);
    }
    return __builtin_fmaf(w.s, acc, __builtin_fmaf(-128.0f, w.s, w.b) * x.sum);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t word = w.q[i >> 2][i & 3];
      const uint32_t lo = pack_bf2_hw((float)(word & 255u), (float)((word >> 8) & 255u));
      const uint32_t hi = pack_bf2_hw((float)((word >> 16) & 255u), (float)(word >> 24));
      acc = dot2(lo, x.p[2 * i], acc);
      acc = dot2(hi, x.p[2 * i + 1], acc);
    }
    return __builtin_fmaf(w.s, acc, w.b * x.sum);
  }
}

// One wave: RP consecutive rows of a gate projection and the matching rows of an up
// projection (SwiGLU) — or of one plain projection — against MT activation rows.  Lane l
// covers input chunks l, l+64, ... (NC chunks).  The body has no data-dependent branches:
// rows past `nrows` reuse the last row, `xrows` arrives clamped to valid rows, lanes past
// the chunk count load chunk 0 and contribute zero, so every load is issued up front.
template <int BITS, int MT, int RP, bool SWIGLU, int NC>
__device__ __forceinline__ void rows_task(const uint32_t *gw, const uint16_t *gs, const uint16_t *gb,
                                          const uint32_t *uw, const uint16_t *us, const uint16_t *ub,
                                          int64_t w_rs, int64_t sb_rs, int nrows, int nchunks,
                                          int group, const uint16_t *x, int64_t ldx,
                                          const int *xrows, int m, uint16_t *out, int64_t ldo,
                                          const int *orows) {
  const int lane = (int)(threadIdx.x & 63);
  float accg[RP][MT], accu[RP][MT];
#pragma unroll
  for (int r = 0; r < RP; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) accg[r][t] = accu[r][t] = 0.0f;
  int xr[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xr[t] = xrows[t];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    const int craw = lane + 64 * cc;
    const bool cv = craw < nchunks;
    const int c = cv ? craw : 0;
    WChunk wg[RP], wu[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      const int rr = r < nrows ? r : nrows - 1;
      load_wchunk<BITS>(wg[r], gw + rr * w_rs, gs + rr * sb_rs, gb + rr * sb_rs, c, group);
      if (SWIGLU) load_wchunk<BITS>(wu[r], uw + rr * w_rs, us + rr * sb_rs, ub + rr * sb_rs, c, group);
    }
    XChunk xc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) load_xchunk<BITS>(xc[t], x + (int64_t)xr[t] * ldx + c * 32);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        const float dg = chunk_dot<BITS>(wg[r], xc[t]);
        accg[r][t] += cv ? dg : 0.0f;
        if (SWIGLU) {
          const float du = chunk_dot<BITS>(wu[r], xc[t]);
          accu[r][t] += cv ? du : 0.0f;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RP; ++r) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const float g = wave_sum_fast(accg[r][t]);
      uint32_t o;
      if (SWIGLU) {
        const float u = wave_sum_fast(accu[r][t]);
        o = swiglu_bf(round_bf(g), round_bf(u));
      } else {
        o = f2bf(g);
      }
      if (lane == 0 && r < nrows && t < m) out[(int64_t)orows[t] * ldo + r] = (uint16_t)o;
    }
  }
}

// rows_task over a few tokens at a time: more tokens run as passes over the same rows (the
// later ones read the codes from L2), which keeps the kernel's registers at the footprint of
// one pass -- kDecodePassTokens tokens for waves of several row pairs, 4 for one row pair --
// and so more waves per SIMD; each token's sums are the same either way.
template <int BITS, int MT, int RP, bool SWIGLU, int NC>
__device__ __forceinline__ void rows_task_q(const uint32_t *gw, const uint16_t *gs, const uint16_t *gb,
                                            const uint32_t *uw, const uint16_t *us, const uint16_t *ub,
                                            int64_t w_rs, int64_t sb_rs, int nrows, int nchunks, int group,
                                            const uint16_t *x, int64_t ldx, const int *xrows, int m, uint16_t *out,
                                            int64_t ldo, const int *orows) {
  constexpr int PT = RP > 1 ? kDecodePassTokens : 4;  // tokens per pass
  if constexpr (MT <= PT) {
    rows_task<BITS, MT, RP, SWIGLU, NC>(gw, gs, gb, uw, us, ub, w_rs, sb_rs, nrows, nchunks, group, x, ldx, xrows,
                                        m, out, ldo, orows);
  } else {
    for (int t0 = 0; t0 < MT; t0 += PT) {
      if (t0 >= m) break;
      rows_task<BITS, PT, RP, SWIGLU, NC>(gw, gs, gb, uw, us, ub, w_rs, sb_rs, nrows, nchunks, group, x, ldx,
                                          xrows + t0, m - t0 < PT ? m - t0 : PT, out, ldo, orows + t0);
    }
  }
}

// ---------------------------------------------------------------- D1: router

// Router GEMV: one wave per expert row, every token.  QB = 0: bf16 weights (forward.rs:59-91,
// matmul); QB = 4 or 8: an affine router (forward.rs:53-58, quantized_linear), its rows
// dequantised per 32-input chunk as the gate/up GEMVs do (chunk_dot).  STEP (the decoder
// step): every workgroup first forms r = bf16(h + a) and the RMS-normalised rows n of the T
// tokens in LDS (the order of add_rms_norm_kernel: rms_* in common.h) and reads its
// activations from there; workgroup 0 also writes r and n for the later kernels.
template <int MT, int NC, bool STEP, int QB>
__global__ __launch_bounds__(256) void decode_router_kernel(const DecodeArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // STEP: n, [T][H]
  __shared__ float wsum[4];
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const int e = blockIdx.x * (int)(blockDim.x >> 6) + wave;
  if (STEP) {
    const int nch = p.H / 8;
    const bool publish = blockIdx.x == 0;
    float part[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      part[t] = 0.0f;
      if (t >= p.T) continue;
      for (int c = threadIdx.x; c < nch; c += 256) {
        const int64_t o = (int64_t)t * p.H + 8 * c;
        const u32x4 r = rms_residual(*(const u32x4 *)(p.h_in + o), p.a_in ? (const u32x4 *)(p.a_in + o) : nullptr);
        *(u32x4 *)(xs + o) = r;
        if (publish) *(u32x4 *)(p.r_out + o) = r;
        part[t] = rms_partial(r, part[t]);
      }
    }
    float inv[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) inv[t] = t < p.T ? rms_inverse(rms_total(part[t], wsum), p.H, p.eps) : 0.0f;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t >= p.T) continue;
      for (int c = threadIdx.x; c < nch; c += 256) {
        const int64_t o = (int64_t)t * p.H + 8 * c;
        const u32x4 n = rms_apply(*(const u32x4 *)(xs + o), *(const u32x4 *)(p.norm_w + 8 * c), inv[t]);
        *(u32x4 *)(xs + o) = n;
        if (publish) *(u32x4 *)(p.x_out + o) = n;
      }
    }
    __syncthreads();
  }
  if (e >= p.E) return;
  const int nchunks = p.H / 32;
  float acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
  if constexpr (QB != 0) {
    const uint32_t *wr = p.rq_w + (int64_t)e * p.rq_w_rs;
    const uint16_t *sr = p.rq_s + (int64_t)e * p.rq_sb_rs, *br = p.rq_b + (int64_t)e * p.rq_sb_rs;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int craw = lane + 64 * cc;
      const bool cv = craw < nchunks;
      const int c = cv ? craw : 0;
      WChunk wc;
      load_wchunk<QB>(wc, wr, sr, br, c, p.rq_group);
      XRaw xr[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int tr = t < p.T ? t : p.T - 1;
        load_xraw(xr[t], (STEP ? xs : p.x) + (int64_t)tr * p.H + c * 32);
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        XChunk xc;
        convert_xchunk<QB>(xc, xr[t]);
        const float d = chunk_dot<QB>(wc, xc);
        acc[t] += cv ? d : 0.0f;
      }
    }
  }
#pragma unroll
  for (int cc = 0; cc < (QB == 0 ? NC : 0); ++cc) {
    const uint16_t *w = p.router_w + (int64_t)e * p.H;
    const int craw = lane + 64 * cc;
    const bool cv = craw < nchunks;
    const int c = cv ? craw : 0;
    const u32x4 *wp = (const u32x4 *)(w + c * 32);
    u32x4 wv[4], xv[MT][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[i] = wp[i];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int tr = t < p.T ? t : p.T - 1;
      const u32x4 *xp = (const u32x4 *)((STEP ? xs : p.x) + (int64_t)tr * p.H + c * 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[t][i] = xp[i];
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) a = dot2(wv[i][j], xv[t][i][j], a);
      acc[t] += cv ? a : 0.0f;
    }
  }
  const float bias = p.router_bias ? bf2f(p.router_bias[e]) : 0.0f;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const float v = wave_sum_fast(acc[t]);
    if (lane == 0 && t < p.T) {
      uint32_t o = f2bf(v);
      if (p.router_bias) o = f2bf(bf2f(o) + bias);
      p.logits[(int64_t)t * p.E + e] = (uint16_t)o;
    }
  }
}

// ---------------------------------------------------------------- D2: route + gate/up

// what decode_route writes to the workspace: the routing (ids, scores, sort, inverse, sorted
// ids, offsets; with a compact page also each assignment's slot and the missing count) and the
// distinct-expert table (count, expert / first row / rows, tokens)
constexpr int kPublishRoute = 1, kPublishTable = 2;

// Where expert e's weights are: e itself, or its compact page slot (an expert with no slot, or
// with a slot past the page, reads slot 0; absent tells the caller to count it).
__device__ __forceinline__ uint32_t page_slot(const DecodeArgs &p, uint32_t e, bool &absent) {
  absent = false;
  if (!p.slot_of_expert) return e;
  const uint32_t s = e < (uint32_t)p.E ? p.slot_of_expert[e] : 0xffffffffu;
  absent = s >= (uint32_t)p.slot_count;
  return absent ? 0u : s;
}

// Routing of the <= 8 tokens from their logits, the stable sort of the <= 64 assignments and
// the table of distinct experts, into LDS; publish (kPublish* bits) selects what is also written
// to the workspace for the later kernels.  EXACT: each token's slice in the order of MLX's CPU
// argpartition (route_token_exact; waves 0 .. route_waves - 1 route, each with
// kSelectWords<PER> words of sel_sh); otherwise the set in ascending id order with no scores
// (route_set8), which gives the same distinct-expert table and rows per expert, but not the
// same slot order -- enough for the table (kPublishTable), not for the routing (kPublishRoute).
template <int MT, int PER, bool EXACT>
__device__ __forceinline__ void decode_route(const DecodeArgs &p, int publish, uint32_t *idx_sh, uint32_t *so_sh,
                                             uint32_t *sid_sh, uint32_t *key_sh, uint32_t (*route_sh)[kDecodeMaxK],
                                             uint16_t *sc_sh, uint32_t *g_expert_sh, uint32_t *g_start_sh,
                                             uint32_t *g_count_sh, uint32_t &ng_sh, uint32_t *sel_sh = nullptr,
                                             int route_waves = 4) {
  constexpr int KM = kDecodeMaxK, AMAX = MT * KM;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const int A = p.A;
  const int nwaves = EXACT ? route_waves : (int)(blockDim.x >> 6);
  for (int t = wave; t < p.T && wave < nwaves; t += nwaves) {
    uint32_t my_idx, my_score;
    if (EXACT) {
      route_token_exact<PER, KM>(p.logits + (int64_t)t * p.E, p.E, p.k, p.normalize,
                                 sel_sh + wave * kSelectWords<PER>, route_sh[wave], my_idx, my_score);
    } else {
      // the set only (the table needs no order and no scores): ascending ids
      uint32_t ids[8];
      route_set8<PER>(p.logits + (int64_t)t * p.E, p.E, p.k, ids);
      my_idx = ids[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) my_idx = lane == i ? ids[i] : my_idx;
      my_score = 0;
    }
    if (lane < p.k) {
      idx_sh[t * p.k + lane] = my_idx;
      sc_sh[t * p.k + lane] = (uint16_t)my_score;
    }
  }
  __syncthreads();
  if (wave == 0) {
    // stable sort by (expert or page slot, assignment): rank = number of smaller keys
    bool absent = false;
    const uint32_t wslot = lane < A ? page_slot(p, idx_sh[lane], absent) : 0u;
    const uint32_t key = lane < A ? (wslot << 6) | (uint32_t)lane : 0xffffffffu;
    key_sh[lane] = key;
    __builtin_amdgcn_wave_barrier();
    // the AMAX >= A keys in broadcast reads, issued before any comparison
    u32x4 kv[AMAX / 4];
#pragma unroll
    for (int b2 = 0; b2 < AMAX / 4; ++b2) kv[b2] = ((const u32x4 *)key_sh)[b2];
    uint32_t rank = 0;
#pragma unroll
    for (int b2 = 0; b2 < AMAX / 4; ++b2)
      rank += (kv[b2][0] < key) + (kv[b2][1] < key) + (kv[b2][2] < key) + (kv[b2][3] < key);
    if (lane < A) {
      so_sh[rank] = (uint32_t)lane;
      sid_sh[rank] = key >> 6;
    }
    __builtin_amdgcn_wave_barrier();
    // distinct experts in ascending order: (expert, first sorted row, count)
    const uint32_t sid = lane < A ? sid_sh[lane] : 0xffffffffu;
    const bool start = lane < A && (lane == 0 || sid != sid_sh[lane - 1]);
    const uint64_t mask = __ballot(start);
    const int gi = __popcll(mask & ((1ull << lane) - 1ull));
    const uint64_t above = lane == 63 ? 0ull : (mask >> (lane + 1));
    const int next = above ? lane + 1 + __ffsll((long long)above) - 1 : A;
    if (start) {
      g_expert_sh[gi] = sid;
      g_start_sh[gi] = (uint32_t)lane;
      g_count_sh[gi] = (uint32_t)(next - lane);
    }
    if (lane == 0) ng_sh = (uint32_t)__popcll(mask);
    if (publish & kPublishRoute) {
      if (lane < A) {
        p.idx[lane] = idx_sh[lane];
        p.scores[lane] = sc_sh[lane];
        p.sorted_order[rank] = (uint32_t)lane;
        p.inverse_order[lane] = rank;
        p.sorted_ids[rank] = key >> 6;
        if (p.slots) p.slots[lane] = wslot;
      }
      const uint64_t absent_lanes = __ballot(lane < A && absent);
      if (p.missing && lane == 0) *p.missing = (uint32_t)__popcll(absent_lanes);
    }
    if (publish & kPublishTable) {
      if (start) {
        p.g_expert[gi] = sid;
        p.g_start[gi] = (uint32_t)lane;
        p.g_count[gi] = (uint32_t)(next - lane);
      }
      if (lane == 0) *p.n_groups = (uint32_t)__popcll(mask);
      // each group's tokens, in sorted-row order, padded with its last (one table read gives
      // the gate/up workgroup its expert and its activation rows)
      if (lane < A) {
        const int g0 = __popcll(mask & ((2ull << lane) - 1ull)) - 1;  // the group of sorted row lane
        const uint64_t at_or_below = mask & ((2ull << lane) - 1ull);
        const int first = 63 - __clzll(at_or_below);  // its first sorted row
        const int i = lane - first;
        const uint64_t later = lane == 63 ? 0ull : (mask >> (lane + 1));
        const bool last = lane + 1 == A || (later & 1ull);
        const uint32_t tok = so_sh[lane] / (uint32_t)p.k;
        if (i < KM) p.g_tokens[g0 * KM + i] = tok;
        if (last)
          for (int j = i + 1; j < KM; ++j) p.g_tokens[g0 * KM + j] = tok;
      }
    }
  }
  __syncthreads();
  if (publish & kPublishRoute) {
    // bucket offsets [buckets + 2] (buckets + 1: trailing out-of-range bucket, empty here)
    for (int e = threadIdx.x; e <= p.buckets + 1; e += (int)blockDim.x) {
      uint32_t c = 0;
#pragma unroll
      for (int i = 0; i < AMAX; ++i) c += (i < A) & (sid_sh[i] < (uint32_t)e);
      p.offsets[e] = e <= p.buckets ? c : (uint32_t)A;
    }
  }
}

// Routing once for a batch of tokens (T >= kDecodeRouteOnceT): one workgroup computes each
// token's top-k set (route_token, one wave per token), the distinct-expert table and each
// group's tokens, and publishes the table; the gate/up kernel's routed workgroups read it
// instead of each recomputing every token's routing.  The table does not depend on the order
// within a token's slice (a token selects an expert at most once, so an expert's sorted rows
// follow its tokens), so the slice in MLX's order -- slow to compute -- is left to a workgroup
// of the gate/up kernel, beside the GEMVs.
template <int MT, int PER>
__global__ __launch_bounds__(64 * MT) void decode_route_kernel(const DecodeArgs p) {
  constexpr int KM = kDecodeMaxK;
  __shared__ uint32_t idx_sh[64], so_sh[64], sid_sh[64];
  __shared__ __attribute__((aligned(16))) uint32_t key_sh[64];
  __shared__ __attribute__((aligned(16))) uint32_t route_sh[MT][KM];
  __shared__ uint16_t sc_sh[64];
  __shared__ uint32_t g_expert_sh[64], g_start_sh[64], g_count_sh[64], ng_sh;
  decode_route<MT, PER, false>(p, kPublishTable, idx_sh, so_sh, sid_sh, key_sh, route_sh, sc_sh, g_expert_sh,
                               g_start_sh, g_count_sh, ng_sh);
}

// Workgroups (x, 0): the shared expert, which needs no routing — x < shared_pair_blocks
// computes 4 (gate row, up row) pairs with the SwiGLU epilogue, x == shared_pair_blocks
// the output gate z.  Workgroups (x, g + 1): rows of the gate/up GEMV of the g-th distinct
// expert for every token routed to it (SwiGLU epilogue).  Without PRE (fewer than
// kDecodeRouteOnceT tokens) every one of them first recomputes the routing's set from the
// logits (route_set8; with two tokens, one wave each, then the stable sort of the assignments
// and the table of distinct experts) — a few microseconds of one wave's work that saves a
// dependent kernel boundary.  With PRE (batches from kDecodeRouteOnceT tokens)
// decode_route_kernel has published the table and the workgroups read it instead.  Either way
// workgroup (shared_pair_blocks + 1, 0) computes the routing in MLX's slot order
// (route_token_exact, one wave per token up to 4 waves) and publishes it for the down kernel,
// next to the GEMVs.  RPW: (gate, up) row pairs per routed wave (more for larger batches:
// fewer, fuller workgroups).
template <int BITS, int MT, int NC, int PER, bool PRE, int RPW>
__global__ __launch_bounds__(256) void decode_gate_up_kernel(const DecodeArgs p) {
  constexpr int KM = kDecodeMaxK;
  __shared__ uint32_t idx_sh[64], so_sh[64], sid_sh[64];
  __shared__ __attribute__((aligned(16))) uint32_t key_sh[64];
  __shared__ __attribute__((aligned(16))) uint32_t route_sh[4][KM];
  __shared__ uint16_t sc_sh[64];
  __shared__ uint32_t g_expert_sh[64], g_start_sh[64], g_count_sh[64], ng_sh;
  __shared__ int rows_sh[MT], orows_sh[MT];
  constexpr int PW = MT < 4 ? MT : 4;  // the publisher's routing waves
  __shared__ uint32_t sel_sh[PW * kSelectWords<PER>];
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int nchunks = p.H / 32;
  if (blockIdx.y == 0 && (int)blockIdx.x == p.shared_pair_blocks + 1) {
    // (with PRE the table is the routing kernel's, identical and already published)
    decode_route<MT, PER, true>(p, PRE ? kPublishRoute : kPublishRoute | kPublishTable, idx_sh, so_sh, sid_sh,
                                key_sh, route_sh, sc_sh, g_expert_sh, g_start_sh, g_count_sh, ng_sh, sel_sh, PW);
    return;
  }
  if (blockIdx.y == 0) {
    if (threadIdx.x < MT) {
      const int t = threadIdx.x < p.T ? threadIdx.x : p.T - 1;
      rows_sh[threadIdx.x] = t;
      orows_sh[threadIdx.x] = p.A + t;
    }
    __syncthreads();
    const int sb = blockIdx.x;
    if (sb < p.shared_pair_blocks) {
      const int r0 = (sb * 4 + wave) * kRowsPerWave;
      if (r0 >= p.Is) return;
      const int nrows = min(kRowsPerWave, p.Is - r0);
      if (p.sg_bits == 4)
        rows_task_q<4, MT, kRowsPerWave, true, NC>(p.sg_w + r0 * p.sg_w_rs, p.sg_s + r0 * p.sg_sb_rs,
                                                 p.sg_b + r0 * p.sg_sb_rs, p.su_w + r0 * p.sg_w_rs,
                                                 p.su_s + r0 * p.sg_sb_rs, p.su_b + r0 * p.sg_sb_rs,
                                                 p.sg_w_rs, p.sg_sb_rs, nrows, nchunks, p.sg_group,
                                                 p.x, p.H, rows_sh, p.T, p.act + r0, p.act_ld,
                                                 orows_sh);
      else
        rows_task_q<8, MT, kRowsPerWave, true, NC>(p.sg_w + r0 * p.sg_w_rs, p.sg_s + r0 * p.sg_sb_rs,
                                                 p.sg_b + r0 * p.sg_sb_rs, p.su_w + r0 * p.sg_w_rs,
                                                 p.su_s + r0 * p.sg_sb_rs, p.su_b + r0 * p.sg_sb_rs,
                                                 p.sg_w_rs, p.sg_sb_rs, nrows, nchunks, p.sg_group,
                                                 p.x, p.H, rows_sh, p.T, p.act + r0, p.act_ld,
                                                 orows_sh);
      return;
    }
    if (sb != p.shared_pair_blocks || wave != 0 || !p.sz_w) return;
    if (p.sz_bits == 4)
      rows_task_q<4, MT, 1, false, NC>(p.sz_w, p.sz_s, p.sz_b, nullptr, nullptr, nullptr, 0, 0, 1,
                                     nchunks, p.sz_group, p.x, p.H, rows_sh, p.T, p.z, 1, rows_sh);
    else
      rows_task_q<8, MT, 1, false, NC>(p.sz_w, p.sz_s, p.sz_b, nullptr, nullptr, nullptr, 0, 0, 1,
                                     nchunks, p.sz_group, p.x, p.H, rows_sh, p.T, p.z, 1, rows_sh);
    return;
  }
  if ((int)blockIdx.x * 4 * RPW >= p.I) return;
  uint32_t e, start, m;
  if (PRE) {
    // the group's table entries, read together with the group count (entries past it are
    // stale and unused)
    const int g = blockIdx.y - 1;
    const uint32_t ng = *p.n_groups;
    e = p.g_expert[g];
    start = p.g_start[g];
    m = p.g_count[g];
    const uint32_t tok = p.g_tokens[g * KM + (threadIdx.x < MT ? threadIdx.x : 0)];
    if (g >= (int)ng) return;
    if (m > (uint32_t)MT) return;  // a token selects an expert at most once: m <= T <= MT
    if (threadIdx.x < MT) {
      const uint32_t i = threadIdx.x < m ? threadIdx.x : m - 1;
      rows_sh[threadIdx.x] = (int)tok;
      orows_sh[threadIdx.x] = (int)(start + i);
    }
  } else if constexpr (MT == 1) {
    // one token: its k experts are the k groups, in ascending id order, each one row (row g,
    // token 0).  Wave 0 computes the set (route_set8: no slot order, scores or sort table) and
    // passes the workgroup's expert on through one LDS word; the other waves wait at the barrier
    // (routing in every wave would crowd the SIMDs' other waves).
    const int g = blockIdx.y - 1;
    if (g >= p.k) return;
    if (wave == 0) {
      uint32_t ids[8];
      route_set8<PER>(p.logits, p.E, p.k, ids);
      uint32_t eg = ids[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) eg = g == i ? ids[i] : eg;
      if (p.slot_of_expert) {
        // a compact page: the g-th of the k slots in (slot, id order) order, the sort's order
        // up to the ties of absent experts (all slot 0, one token: equal rows)
        const int ln = (int)(threadIdx.x & 63);
        uint32_t mine = ids[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mine = ln == i ? ids[i] : mine;
        bool absent;
        const uint32_t sl = ln < p.k ? page_slot(p, mine, absent) : 0xffffffffu;
        int rank = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t si = (uint32_t)__builtin_amdgcn_readlane((int)sl, i);
          rank += (i < p.k) && (si < sl || (si == sl && i < ln));
        }
        const uint64_t hit = __ballot(ln < p.k && rank == g);
        eg = (uint32_t)__builtin_amdgcn_readlane((int)sl, (int)__ffsll((long long)hit) - 1);
      }
      if ((threadIdx.x & 63) == 0) g_expert_sh[0] = eg;
    }
    __syncthreads();
    e = g_expert_sh[0];
    start = (uint32_t)g;
    m = 1;
  } else {
    decode_route<MT, PER, false>(p, 0, idx_sh, so_sh, sid_sh, key_sh, route_sh, sc_sh, g_expert_sh,
                                 g_start_sh, g_count_sh, ng_sh);
    const int g = blockIdx.y - 1;
    if (g >= (int)ng_sh) return;
    e = g_expert_sh[g];
    start = g_start_sh[g];
    m = g_count_sh[g];
    if (m > (uint32_t)MT) return;  // a token selects an expert at most once: m <= T <= MT
    if (threadIdx.x < MT) {
      const uint32_t i = threadIdx.x < m ? threadIdx.x : m - 1;
      rows_sh[threadIdx.x] = (int)(so_sh[start + i] / (uint32_t)p.k);
      orows_sh[threadIdx.x] = (int)(start + i);
    }
  }
  const int xrow0 = 0, orow0 = (int)start;  // the single-token path's row and output row
  constexpr bool kOne = !PRE && MT == 1;
  if (!kOne) __syncthreads();
  const int *xrows = kOne ? &xrow0 : rows_sh, *orows = kOne ? &orow0 : orows_sh;
  const int r0 = (blockIdx.x * 4 + wave) * RPW;
  if (r0 >= p.I) return;
  const int nrows = min(RPW, p.I - r0);
  const int64_t wo = (int64_t)e * p.gu_w_es + (int64_t)r0 * p.gu_w_rs;
  const int64_t so = (int64_t)e * p.gu_sb_es + (int64_t)r0 * p.gu_sb_rs;
  // the expert's m <= MT tokens: the smallest token count instantiated that covers them (each
  // token's sums do not depend on it)
  auto routed_rows = [&](auto mt_tag) {
    constexpr int M2 = decltype(mt_tag)::value;
    rows_task_q<BITS, M2, RPW, true, NC>(p.gate_w + wo, p.gate_s + so, p.gate_b + so, p.up_w + wo,
                                                p.up_s + so, p.up_b + so, p.gu_w_rs, p.gu_sb_rs, nrows, nchunks,
                                                p.gu_group, p.x, p.H, xrows, (int)m, p.act + r0, p.act_ld,
                                                orows);
  };
  if (m <= 1) routed_rows(std::integral_constant<int, 1>());
  else if (MT > 2 && m <= 2) routed_rows(std::integral_constant<int, (MT > 2 ? 2 : MT)>());
  else if (MT > 4 && m <= 4) routed_rows(std::integral_constant<int, (MT > 4 ? 4 : MT)>());
  else routed_rows(std::integral_constant<int, MT>());
}

// ---------------------------------------------------------------- D3: down + combine

// One workgroup per (4 R output rows, token).  The token's k experts and, in a block with a
// shared expert (SH), the shared expert are P = kDecodeMaxK (+ 1) participant rows per output
// row, dealt to NW waves so that none loads a participant it masks out: one per wave up to
// four tokens; beyond, with the shared expert 3 waves of 3 (wave w: participants w, w+3,
// w+6), without it 4 waves of 2 (w, w+4).
// Quarter q of a wave (one DPP row of 16 lanes) takes output rows (4x + q) R .. + R and its 16 lanes split the input chunks (lane l16 takes chunks l16,
// l16+16, ...); a participant's activation chunk is loaded once for its R rows.  The rounded
// participant values meet in LDS, where wave 0 forms the weighted combine (slot order) and the
// shared expert's gated add, lane l16 < R of quarter q for row (4x + q) R + l16.  Larger
// batches take R > 1: fewer, longer workgroups (every workgroup's dependent chain of index
// and weight loads is paid once per R rows).  Branch-free: participants past k, or a missing
// shared expert, reuse slot 0's rows and are masked out.
template <int BITS, int NC, bool SORTED, int R, bool SH, int NW>
__global__ __launch_bounds__(64 * NW) void decode_down_kernel(const DecodeArgs p) {
  constexpr int KM = kDecodeMaxK, P = SH ? KM + 1 : KM, PW = (P + NW - 1) / NW;
  __shared__ float vals[4][R][NW * PW];
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, l16 = lane & 15, q = lane >> 4;
  const int t = blockIdx.y, h0 = (blockIdx.x * 4 + q) * R;
  const bool has_shared = SH && p.Is > 0;
  // loads the combine needs, issued first (a missing shared expert reads a score instead)
  const uint16_t zbits = has_shared ? p.z[t] : p.scores[0];
  const int hc = h0 + (l16 < R ? l16 : 0);  // this lane's row in the combine
  const uint16_t rbits = p.ffn_out ? p.r_out[(int64_t)t * p.H + hc] : 0;  // the decoder step's residual
  float sc[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) sc[j] = bf2f(p.scores[t * p.k + (j < p.k ? j : p.k - 1)]);

  // participant rows, selected without branches
  const uint32_t *sd_w = has_shared ? p.sd_w : p.down_w;
  const uint16_t *sd_s = has_shared ? p.sd_s : p.down_s;
  const uint16_t *sd_b = has_shared ? p.sd_b : p.down_b;
  const int64_t sd_w_rs = has_shared ? p.sd_w_rs : p.dn_w_rs;
  const int64_t sd_sb_rs = has_shared ? p.sd_sb_rs : p.dn_sb_rs;
  const int sd_nch = has_shared ? p.Is / 32 : p.I / 32;
  const int sd_group = has_shared ? p.sd_group : p.dn_group;
  uint32_t e[PW], r[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int j = wave + NW * i;
    const int a = t * p.k + (j < p.k ? j : 0);
    e[i] = p.slots ? p.slots[a] : p.idx[a];  // the weights' expert or page slot
    r[i] = p.inverse_order[a];
  }
  const uint32_t *wrow[PW];
  const uint16_t *srow[PW], *brow[PW];
  const uint16_t *xrow[PW];
  int64_t wrs[PW], sbrs[PW];
  int nch[PW], grp[PW];
  uint32_t orow[PW];
  bool live[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int j = wave + NW * i;
    const bool shared = j == KM && has_shared;
    live[i] = (j < KM && j < p.k) || shared;
    orow[i] = shared ? (uint32_t)(p.A + t) : r[i];
    const uint32_t *wb = shared ? sd_w : p.down_w + (int64_t)e[i] * p.dn_w_es;
    const uint16_t *sb = shared ? sd_s : p.down_s + (int64_t)e[i] * p.dn_sb_es;
    const uint16_t *bb = shared ? sd_b : p.down_b + (int64_t)e[i] * p.dn_sb_es;
    wrs[i] = shared ? sd_w_rs : p.dn_w_rs;
    sbrs[i] = shared ? sd_sb_rs : p.dn_sb_rs;
    wrow[i] = wb + (int64_t)h0 * wrs[i];
    srow[i] = sb + (int64_t)h0 * sbrs[i];
    brow[i] = bb + (int64_t)h0 * sbrs[i];
    xrow[i] = p.act + (int64_t)orow[i] * p.act_ld;
    nch[i] = shared ? sd_nch : p.I / 32;
    grp[i] = shared ? sd_group : p.dn_group;
  }
  float acc[PW][R];
#pragma unroll
  for (int i = 0; i < PW; ++i)
#pragma unroll
    for (int rr = 0; rr < R; ++rr) acc[i][rr] = 0.0f;
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    const int craw = l16 + 16 * cc;
    // every load of the chunk step first, then the arithmetic
    WChunk wch[PW][R];
    XRaw xr[PW];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int c = craw < nch[i] ? craw : 0;
#pragma unroll
      for (int rr = 0; rr < R; ++rr)
        load_wchunk<BITS>(wch[i][rr], wrow[i] + rr * wrs[i], srow[i] + rr * sbrs[i], brow[i] + rr * sbrs[i], c,
                          grp[i]);
      load_xraw(xr[i], xrow[i] + c * 32);
    }
    // keep the scheduler from interleaving the first participant's arithmetic (and its
    // waits) with the later participants' loads
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      XChunk xc;
      convert_xchunk<BITS>(xc, xr[i]);
#pragma unroll
      for (int rr = 0; rr < R; ++rr) {
        const float d = chunk_dot<BITS>(wch[i][rr], xc);
        acc[i][rr] += craw < nch[i] ? d : 0.0f;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < PW; ++i)
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const float v = round_bf(row_sum(acc[i][rr]));
      if (l16 == rr) {
        vals[q][rr][wave + NW * i] = v;
        if (live[i]) p.down_out[(int64_t)orow[i] * p.H + h0 + rr] = (uint16_t)f2bf(v);
      }
    }
  __syncthreads();
  if (wave != 0 || l16 >= R) return;
  float v[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) v[j] = vals[q][l16][j];
  const uint32_t sparse = combine_element<SORTED, KM>(v, sc, p.k);
  uint32_t out = sparse;
  if (has_shared) out = shared_gated_add(sparse, vals[q][l16][KM], round_bf(det_sigmoid(bf2f(zbits))));
  p.sparse[(int64_t)t * p.H + hc] = (uint16_t)sparse;
  p.y[(int64_t)t * p.H + hc] = (uint16_t)out;
  if (p.ffn_out) p.ffn_out[(int64_t)t * p.H + hc] = (uint16_t)f2bf(bf2f(rbits) + bf2f(out));
}

// threads per workgroup (256 unless given); ev (nullable) = {start, stop} events recorded around the kernel itself
template <typename Kernel>
void launch_timed(Kernel kernel, dim3 grid, hipStream_t s, const hipEvent_t *ev, const DecodeArgs &a, int threads = 256) {
  if (ev)
    hipExtLaunchKernelGGL(kernel, grid, dim3(threads), 0, s, ev[0], ev[1], 0, a);
  else
    hipLaunchKernelGGL(kernel, grid, dim3(threads), 0, s, a);
}

template <int BITS, int MT, int NC, int PER, int RPW>
void launch_gate_up_rpw(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  // x: routed row blocks, or the shared expert's pair blocks and its output-gate block
  const int routed_x = (a.I + 4 * RPW - 1) / (4 * RPW);
  // x <= shared_pair_blocks: the shared expert; shared_pair_blocks + 1: the routing publisher
  const int shared_x = a.shared_pair_blocks + 2;
  const dim3 grid(std::max(routed_x, shared_x), a.max_groups + 1);
  if (a.T >= kDecodeRouteOnceT)
    launch_timed(decode_gate_up_kernel<BITS, MT, NC, PER, true, RPW>, grid, s, ev, a);
  else
    launch_timed(decode_gate_up_kernel<BITS, MT, NC, PER, false, RPW>, grid, s, ev, a);
}

template <int BITS, int MT, int NC, int PER>
void launch_gate_up_per(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  // one row pair per routed wave for a single token (the chip has wave slots to spare); a
  // batch selects up to 8x more distinct experts, so each wave takes more rows
  if (MT <= 1) launch_gate_up_rpw<BITS, MT, NC, PER, kRowsPerWave>(a, s, ev);
  else if (MT <= 2) launch_gate_up_rpw<BITS, MT, NC, PER, 2>(a, s, ev);
  else launch_gate_up_rpw<BITS, MT, NC, PER, 4>(a, s, ev);
}

// one workgroup, one wave per token slot and at least 4 (the E + 2 expert offsets are spread
// over every thread of the block)
template <int MT, int PER>
void launch_route_per(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  constexpr int W = MT > 4 ? MT : 4;
  if (ev)
    hipExtLaunchKernelGGL((decode_route_kernel<W, PER>), dim3(1), dim3(64 * W), 0, s, ev[0], ev[1], 0, a);
  else
    hipLaunchKernelGGL((decode_route_kernel<W, PER>), dim3(1), dim3(64 * W), 0, s, a);
}

template <int MT>
void launch_route_mt(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  const int per = (a.E + 63) / 64;
  if (per <= 1) launch_route_per<MT, 1>(a, s, ev);
  else if (per <= 2) launch_route_per<MT, 2>(a, s, ev);
  else if (per <= 4) launch_route_per<MT, 4>(a, s, ev);
  else if (per <= 8) launch_route_per<MT, 8>(a, s, ev);
  else launch_route_per<MT, 16>(a, s, ev);
}

template <int BITS, int MT, int NC>
void launch_gate_up_nc(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  const int per = (a.E + 63) / 64;
  if (per <= 1) launch_gate_up_per<BITS, MT, NC, 1>(a, s, ev);
  else if (per <= 2) launch_gate_up_per<BITS, MT, NC, 2>(a, s, ev);
  else if (per <= 4) launch_gate_up_per<BITS, MT, NC, 4>(a, s, ev);
  else if (per <= 8) launch_gate_up_per<BITS, MT, NC, 8>(a, s, ev);
  else launch_gate_up_per<BITS, MT, NC, 16>(a, s, ev);
}

template <int BITS, int NC, int R, bool SH, int NW>
void launch_down_w(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev, bool sorted) {
  const dim3 grid(a.H / (4 * R), a.T);
  if (sorted) launch_timed(decode_down_kernel<BITS, NC, true, R, SH, NW>, grid, s, ev, a, 64 * NW);
  else launch_timed(decode_down_kernel<BITS, NC, false, R, SH, NW>, grid, s, ev, a, 64 * NW);
}

template <int BITS, int NC, int R>
void launch_down_r(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  // routing.rs:13 / resident_execution.rs:86-95: sorted reduction iff A >= 64; a verification
  // window keeps the unsorted one (resident_execution.rs:161-162)
  // one wave per participant up to kDecodeDownWideT tokens, then 3 waves of 3 (4 of 2)
  const bool sorted = a.A >= 64 && !a.unsorted, wide = a.T <= kDecodeDownWideT;
  if (a.Is > 0) {
    if (wide) launch_down_w<BITS, NC, R, true, 9>(a, s, ev, sorted);
    else launch_down_w<BITS, NC, R, true, 3>(a, s, ev, sorted);
  } else {
    if (wide) launch_down_w<BITS, NC, R, false, 8>(a, s, ev, sorted);
    else launch_down_w<BITS, NC, R, false, 4>(a, s, ev, sorted);
  }
}

template <int BITS, int NC>
void launch_down_nc(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  // output rows per quarter-wave by batch size (H is a multiple of 32, so 4 R divides it);
  // longer rows keep one row per quarter and 8-bit codes at most two (their code registers)
  const int r = a.T <= kDecodeDownR1T ? 1 : a.T <= kDecodeDownR2T ? 2 : 4;
  if constexpr (NC > 1) {
    launch_down_r<BITS, NC, 1>(a, s, ev);
  } else if constexpr (BITS == 8) {
    if (r == 1) launch_down_r<BITS, NC, 1>(a, s, ev);
    else launch_down_r<BITS, NC, 2>(a, s, ev);
  } else {
    if (r == 1) launch_down_r<BITS, NC, 1>(a, s, ev);
    else if (r == 2) launch_down_r<BITS, NC, 2>(a, s, ev);
    else launch_down_r<BITS, NC, 4>(a, s, ev);
  }
}

template <int BITS, int MT>
void launch_gate_up_mt(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  if (a.H <= 2048) launch_gate_up_nc<BITS, MT, 1>(a, s, ev);
  else launch_gate_up_nc<BITS, MT, 2>(a, s, ev);
}

template <int BITS>
void launch_down(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  if (std::max(a.I, a.Is) <= 512) launch_down_nc<BITS, 1>(a, s, ev);
  else launch_down_nc<BITS, 2>(a, s, ev);
}

template <int MT, int NC, int QB>
void launch_router_nc(const DecodeArgs &a, int blocks, hipStream_t s, const hipEvent_t *ev) {
  if (!a.norm_w) {
    // one wave per workgroup: the E rows' loads come from E CUs rather than E / 4
    if (ev)
      hipExtLaunchKernelGGL(decode_router_kernel<MT, NC, false, QB>, dim3(a.E), dim3(64), 0, s, ev[0], ev[1], 0, a);
    else
      hipLaunchKernelGGL((decode_router_kernel<MT, NC, false, QB>), dim3(a.E), dim3(64), 0, s, a);
    return;
  }
  const size_t lds = (size_t)a.T * a.H * 2;
  if (ev)
    hipExtLaunchKernelGGL(decode_router_kernel<MT, NC, true, QB>, dim3(blocks), dim3(256), lds, s, ev[0], ev[1], 0, a);
  else
    hipLaunchKernelGGL((decode_router_kernel<MT, NC, true, QB>), dim3(blocks), dim3(256), lds, s, a);
}

template <int MT, int QB>
void launch_router_q(const DecodeArgs &a, int blocks, hipStream_t s, const hipEvent_t *ev) {
  if (a.H <= 2048) launch_router_nc<MT, 1, QB>(a, blocks, s, ev);
  else launch_router_nc<MT, 2, QB>(a, blocks, s, ev);
}

template <int MT>
void launch_router(const DecodeArgs &a, int blocks, hipStream_t s, const hipEvent_t *ev) {
  if (a.router_w) launch_router_q<MT, 0>(a, blocks, s, ev);
  else if (a.rq_bits == 8) launch_router_q<MT, 8>(a, blocks, s, ev);
  else launch_router_q<MT, 4>(a, blocks, s, ev);
}

}  // namespace

// gate/up launch of one (code width, token count) variant (decode_gate_up.hip)
template <int BITS, int MT>
void launch_decode_gate_up(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev);

}  // namespace astro
