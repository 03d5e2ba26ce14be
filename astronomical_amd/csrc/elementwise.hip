// Bandwidth-bound pieces of the block: SwiGLU, the weighted expert combine with the
// shared expert's gated add, a skinny quantized GEMV (the shared expert's 2048 -> 1 output
// gate), and the small index / add operations of the paged callers (page slot remap,
// assignment gather, bf16 add).
#include "common.h"
#include "kernels.h"

namespace astro {

namespace {

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *__restrict__ g,
                                                     const uint16_t *__restrict__ u, int64_t n,
                                                     uint16_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (uint16_t)swiglu_bf(bf2f(g[i]), bf2f(u[i]));
}

// Accumulate one expert row into the 8 running sums: sorted rounding (fp32 fma of
// out*score, weighted_sum.rs:16-33) or unsorted rounding (bf16 product, then fp32 add,
// weighted_sum.rs:112-119).
template <bool SORTED>
__device__ __forceinline__ void accumulate8(float acc[8], const float v[8], float s) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (SORTED) acc[i] = __builtin_fmaf(v[i], s, acc[i]);
    else acc[i] = acc[i] + round_bf(v[i] * s);
  }
}

__device__ __forceinline__ void unpack8(float v[8], const u32x4 q) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf_lo(q[i]);
    v[2 * i + 1] = bf_hi(q[i]);
  }
}

// y[t][d] for 8 consecutive d per thread.  Row of assignment (t, j): inverse_order[t*k+j]
// (or t*k+j when inverse_order is null); slots are summed in slot order with one bf16
// rounding at the end.  Then, with a shared expert:
// y = bf16(sparse + bf16(shared * bf16(sigmoid(z)))) (output_combination.rs:40-42).
// K > 0: the top-k width is K and every index, score and row load is issued before the
// first use; K == 0: any k, element loads (no alignment or width assumptions).
template <bool SORTED, int K>
__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t *__restrict__ rows, const uint32_t *__restrict__ inverse_order,
    const uint16_t *__restrict__ scores, int T, int k, int D,
    const uint16_t *__restrict__ shared_out, const uint16_t *__restrict__ gate_logits,
    uint16_t *__restrict__ sparse_out, uint16_t *__restrict__ y) {
#pragma clang fp contract(off)
  const int chunks = (D + 7) >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)T * chunks) return;
  const int t = (int)(gid / chunks), d0 = (int)(gid % chunks) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (K > 0) {
    uint32_t inv[K > 0 ? K : 1];
    float sc[K > 0 ? K : 1];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int64_t a = (int64_t)t * K + j;
      inv[j] = inverse_order ? inverse_order[a] : (uint32_t)a;
      sc[j] = bf2f(scores[a]);
    }
    u32x4 q[K > 0 ? K : 1];
#pragma unroll
    for (int j = 0; j < K; ++j) q[j] = *(const u32x4 *)(rows + (int64_t)inv[j] * D + d0);
#pragma unroll
    for (int j = 0; j < K; ++j) {
      float v[8];
      unpack8(v, q[j]);
      accumulate8<SORTED>(acc, v, sc[j]);
    }
  } else {
    for (int j = 0; j < k; ++j) {
      const int64_t a = (int64_t)t * k + j;
      const int64_t r = inverse_order ? (int64_t)inverse_order[a] : a;
      const uint16_t *src = rows + r * D + d0;
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = d0 + i < D ? bf2f(src[i]) : 0.f;
      accumulate8<SORTED>(acc, v, bf2f(scores[a]));
    }
  }
  uint32_t outb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) outb[i] = f2bf(acc[i]);
  const bool full = d0 + 8 <= D;
  if (sparse_out) {
    uint16_t *dst = sparse_out + (int64_t)t * D + d0;
    if (K > 0) {
      *(u32x4 *)dst = u32x4{outb[0] | (outb[1] << 16), outb[2] | (outb[3] << 16),
                            outb[4] | (outb[5] << 16), outb[6] | (outb[7] << 16)};
    } else {
      for (int i = 0; i < 8; ++i)
        if (d0 + i < D) dst[i] = (uint16_t)outb[i];
    }
  }
  if (shared_out) {
    const float gate = round_bf(det_sigmoid(bf2f(gate_logits[t])));
    const uint16_t *so = shared_out + (int64_t)t * D + d0;
    float sv[8];
    if (K > 0) {
      unpack8(sv, *(const u32x4 *)so);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = d0 + i < D ? bf2f(so[i]) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) outb[i] = f2bf(bf2f(outb[i]) + round_bf(sv[i] * gate));
  }
  uint16_t *dst = y + (int64_t)t * D + d0;
  if (K > 0 && full) {
    *(u32x4 *)dst = u32x4{outb[0] | (outb[1] << 16), outb[2] | (outb[3] << 16),
                          outb[4] | (outb[5] << 16), outb[6] | (outb[7] << 16)};
  } else {
    for (int i = 0; i < 8; ++i)
      if (d0 + i < D) dst[i] = (uint16_t)outb[i];
  }
}

__global__ __launch_bounds__(256) void combine_shared_kernel(
    const uint16_t *__restrict__ sparse, const uint16_t *__restrict__ shared_out,
    const uint16_t *__restrict__ gate_logits, int T, int D, uint16_t *__restrict__ y) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)T * D) return;
  const int t = (int)(i / D);
  const float gate = round_bf(det_sigmoid(bf2f(gate_logits[t])));
  y[i] = (uint16_t)f2bf(bf2f(sparse[i]) + round_bf(bf2f(shared_out[i]) * gate));
}

// One wave per (token, output row) (qgemv_row_wave).
template <int BITS>
__global__ __launch_bounds__(256) void qgemv_rows_kernel(
    const uint16_t *__restrict__ x, int T, int K, const uint32_t *__restrict__ w,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ bi, int N, int group,
    uint16_t *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (item >= T * N) return;
  const int t = item / N, n = item % N;
  const float acc = qgemv_row_wave<BITS>(x + (int64_t)t * K, K, w + (int64_t)n * (K * BITS / 32),
                                         sc + (int64_t)n * (K / group), bi + (int64_t)n * (K / group), group);
  if (lane == 0) out[(int64_t)t * N + n] = (uint16_t)f2bf(acc);
}

template <bool SORTED, int K>
void launch_combine_t(const uint16_t *rows, const uint32_t *inverse_order, const uint16_t *scores,
                      int T, int k, int D, const uint16_t *shared_out, const uint16_t *gate_logits,
                      uint16_t *sparse_out, uint16_t *y, hipStream_t s) {
  const int64_t threads = (int64_t)T * ((D + 7) / 8);
  hipLaunchKernelGGL((combine_kernel<SORTED, K>), dim3((unsigned)((threads + 255) / 256)), dim3(256),
                     0, s, rows, inverse_order, scores, T, k, D, shared_out, gate_logits,
                     sparse_out, y);
}

template <bool SORTED>
void launch_combine_s(const uint16_t *rows, const uint32_t *inverse_order, const uint16_t *scores,
                      int T, int k, int D, const uint16_t *shared_out, const uint16_t *gate_logits,
                      uint16_t *sparse_out, uint16_t *y, hipStream_t s) {
  // the unrolled variants need 16-byte aligned rows of a width divisible by 8
  const bool vec = (D % 8) == 0 && ((uintptr_t)rows % 16) == 0 && ((uintptr_t)y % 16) == 0 &&
                   (!sparse_out || ((uintptr_t)sparse_out % 16) == 0) &&
                   (!shared_out || ((uintptr_t)shared_out % 16) == 0);
  if (vec && k == 8)
    launch_combine_t<SORTED, 8>(rows, inverse_order, scores, T, k, D, shared_out, gate_logits, sparse_out, y, s);
  else if (vec && k == 4)
    launch_combine_t<SORTED, 4>(rows, inverse_order, scores, T, k, D, shared_out, gate_logits, sparse_out, y, s);
  else
    launch_combine_t<SORTED, 0>(rows, inverse_order, scores, T, k, D, shared_out, gate_logits, sparse_out, y, s);
}

// page slot of every assignment: slots[a] = slot_of_expert[ids[a]]; an id past the map or
// a slot marked absent (0xffffffff) counts into *missing and reads slot 0 instead, so every
// later weight access stays inside the page
__global__ __launch_bounds__(256) void remap_slots_kernel(const uint32_t *__restrict__ ids, int n,
                                                          const uint32_t *__restrict__ slot_of_expert,
                                                          int experts, uint32_t *__restrict__ slots,
                                                          uint32_t *__restrict__ missing) {
  const int a = blockIdx.x * blockDim.x + threadIdx.x;
  if (a >= n) return;
  const uint32_t e = ids[a];
  uint32_t s = e < (uint32_t)experts ? slot_of_expert[e] : 0xffffffffu;
  if (s == 0xffffffffu) {
    if (missing) atomicAdd(missing, 1u);
    s = 0;
  }
  slots[a] = s;
}

// out_ids[i] = ids[positions[i]], out_scores[i] = scores[positions[i]]
__global__ __launch_bounds__(256) void gather_assignments_kernel(
    const uint32_t *__restrict__ ids, const uint16_t *__restrict__ scores,
    const uint32_t *__restrict__ positions, int n, uint32_t *__restrict__ out_ids,
    uint16_t *__restrict__ out_scores) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t a = positions[i];
  if (out_ids) out_ids[i] = ids[a];
  if (out_scores) out_scores[i] = scores[a];
}

// a few words set to zero (a kernel, so that callers may capture it in a graph)
__global__ __launch_bounds__(64) void zero_u32_kernel(uint32_t *__restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += 64) p[i] = 0;
}

// bf16 + bf16 -> bf16: the fp32 sum rounded to nearest even (MLX add on bf16 arrays)
__global__ __launch_bounds__(256) void add_bf16_kernel(const uint16_t *__restrict__ a,
                                                       const uint16_t *__restrict__ b, int64_t n,
                                                       uint16_t *__restrict__ out) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (uint16_t)f2bf(bf2f(a[i]) + bf2f(b[i]));
}

// The decoder's RMSNorm input of the block (decoder_layer_forward.rs:111-116 with MLX
// fast::rms_norm): r = bf16(h + a) (a may be null: r = h), n = bf16(w * bf16(r * inv)) with
// inv = 1 / sqrt(mean(r^2) + eps) in fp32 (IEEE sqrt and division).  mean(r^2) in a fixed
// order the host oracle and the decode router kernel repeat (rms_partial / rms_total in
// common.h): thread j of 256 owns the 8-element chunks j, j + 256, ... and sums their r^2 in
// element order; each wave combines its lanes by the canonical butterfly and the four wave sums
// add as (w0 + w1) + (w2 + w3).  One workgroup per token row; H a multiple of 8.
template <int PER>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(const uint16_t *__restrict__ h,
                                                           const uint16_t *__restrict__ a,
                                                           const uint16_t *__restrict__ w, float eps,
                                                           int H, uint16_t *__restrict__ r_out,
                                                           uint16_t *__restrict__ n_out) {
#pragma clang fp contract(off)
  __shared__ float wsum[4];
  const int64_t row = (int64_t)blockIdx.x * H;
  const int tid = threadIdx.x;
  const int nch = H / 8;
  u32x4 rv[PER];
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = tid + 256 * i;
    rv[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < nch) {
      rv[i] = rms_residual(*(const u32x4 *)(h + row + 8 * c), a ? (const u32x4 *)(a + row + 8 * c) : nullptr);
      if (r_out) *(u32x4 *)(r_out + row + 8 * c) = rv[i];
      part = rms_partial(rv[i], part);
    }
  }
  const float inv = rms_inverse(rms_total(part, wsum), H, eps);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = tid + 256 * i;
    if (c < nch) *(u32x4 *)(n_out + row + 8 * c) = rms_apply(rv[i], *(const u32x4 *)(w + 8 * c), inv);
  }
}

// tanh(x) = sign(x) (1 - 2 / (e^(2|x|) + 1)) on det_expf: the same steps on the host give the
// same bits
__device__ __forceinline__ float det_tanh(float x) {
#pragma clang fp contract(off)
  const float ax = __builtin_fabsf(x);
  const float t = 1.0f - 2.0f / (det_expf(2.0f * ax) + 1.0f);
  return x != x ? x : __builtin_copysignf(t, x);
}

// route_laguna_experts (laguna/moe/router.rs:29-94) in the order of the reference's CPU
// selection select_laguna_router_experts (router_selection.rs:59-116): one wave per token;
// expert e scores s = sigmoid(l) of its fp32 logit l (after l = tanh(l / c) c when the softcap
// c > 0); the k experts of largest s + bias (f32 total order, ties to the lower expert id) in
// that descending order; their unbiased s, divided by the in-order fp32 sum of the k when
// normalize and that sum is positive.  Keys: (total-order bits of s + bias) << 32 | ~e.
template <int PER>
__global__ __launch_bounds__(256) void laguna_route_kernel(const uint16_t *__restrict__ logits, int T,
                                                           int E, int k, const float *__restrict__ bias,
                                                           float softcap, int normalize,
                                                           uint32_t *__restrict__ idx,
                                                           float *__restrict__ scores) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  const uint16_t *l = logits + (int64_t)t * E;
  auto score = [&](int e) {
    float v = bf2f(l[e]);
    if (softcap > 0.0f) v = det_tanh(v / softcap) * softcap;
    return det_sigmoid(v);
  };
  uint64_t cand[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const int ec = e < E ? e : E - 1;
    const float sel = score(ec) + (bias ? bias[ec] : 0.0f);
    uint32_t b = __float_as_uint(sel);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    cand[i] = e < E ? ((uint64_t)b << 32) | (uint64_t)(0xffffffffu - (uint32_t)e) : 0ull;
  }
  // per-lane descending order (odd-even transposition network)
#pragma unroll
  for (int pass = 0; pass < PER; ++pass)
#pragma unroll
    for (int i = pass & 1; i + 1 < PER; i += 2) {
      const uint64_t hi = cand[i] > cand[i + 1] ? cand[i] : cand[i + 1];
      const uint64_t lo = cand[i] > cand[i + 1] ? cand[i + 1] : cand[i];
      cand[i] = hi;
      cand[i + 1] = lo;
    }
  uint64_t mine = 0;
  for (int r = 0; r < k; ++r) {
    uint64_t top = cand[0];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)top, off, kWave);
      const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(top >> 32), off, kWave);
      const uint64_t o = ((uint64_t)hi << 32) | lo;
      top = o > top ? o : top;
    }
    const bool hit = cand[0] == top;
#pragma unroll
    for (int i = 0; i + 1 < PER; ++i) cand[i] = hit ? cand[i + 1] : cand[i];
    cand[PER - 1] = hit ? 0ull : cand[PER - 1];
    mine = lane == r ? top : mine;
  }
  const uint32_t e = 0xffffffffu - (uint32_t)mine;
  float s = lane < k ? score(e) : 0.0f;
  if (normalize) {
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), j));
    if (sum > 0.0f) s = s / sum;
  }
  if (lane < k) {
    idx[(int64_t)t * k + lane] = e;
    scores[(int64_t)t * k + lane] = s;
  }
}

// Every fp32 bit pattern: the conversion the kernels round with (f2bf) against the rounding
// on the bit pattern (f2bf_bits); mismatches counted into *count (zeroed by the first kernel).
constexpr int kSelfTestPerThread = 1024;
__global__ void zero_u64_kernel(unsigned long long *p) { *p = 0; }
__global__ __launch_bounds__(256) void selftest_bf16_kernel(unsigned long long *count) {
  const uint32_t base = ((uint32_t)blockIdx.x * 256u + threadIdx.x) * (uint32_t)kSelfTestPerThread;
  unsigned int bad = 0;
  for (int j = 0; j < kSelfTestPerThread; ++j) {
    const float f = __uint_as_float(base + (uint32_t)j);
    bad += f2bf(f) != f2bf_bits(f);
  }
  if (bad) atomicAdd(count, (unsigned long long)bad);
}

}  // namespace

hipError_t launch_add_rms_norm(const uint16_t *h, const uint16_t *a, const uint16_t *w, float eps, int T,
                               int H, uint16_t *r_out, uint16_t *n_out, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  const int per = (H / 8 + 255) / 256;
#define ASTRO_RMS(P) hipLaunchKernelGGL(add_rms_norm_kernel<P>, dim3(T), dim3(256), 0, s, h, a, w, eps, H, r_out, n_out)
  if (per <= 1) ASTRO_RMS(1);
  else if (per <= 2) ASTRO_RMS(2);
  else ASTRO_RMS(4);
#undef ASTRO_RMS
  return hipGetLastError();
}

hipError_t launch_route_laguna(const uint16_t *logits, int T, int E, int k, const float *bias, float softcap,
                               int normalize, uint32_t *idx, float *scores, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  const int per = (E + 63) / 64;
  const dim3 grid((T + 3) / 4), block(256);
#define ASTRO_LAG(P) hipLaunchKernelGGL(laguna_route_kernel<P>, grid, block, 0, s, logits, T, E, k, bias, softcap, normalize, idx, scores)
  if (per <= 1) ASTRO_LAG(1);
  else if (per <= 2) ASTRO_LAG(2);
  else if (per <= 4) ASTRO_LAG(4);
  else if (per <= 8) ASTRO_LAG(8);
  else ASTRO_LAG(16);
#undef ASTRO_LAG
  return hipGetLastError();
}

hipError_t launch_remap_slots(const uint32_t *ids, int n, const uint32_t *slot_of_expert, int experts,
                              uint32_t *slots, uint32_t *missing, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(remap_slots_kernel, dim3((n + 255) / 256), dim3(256), 0, s, ids, n, slot_of_expert,
                     experts, slots, missing);
  return hipGetLastError();
}

hipError_t launch_gather_assignments(const uint32_t *ids, const uint16_t *scores,
                                     const uint32_t *positions, int n, uint32_t *out_ids,
                                     uint16_t *out_scores, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_assignments_kernel, dim3((n + 255) / 256), dim3(256), 0, s, ids, scores,
                     positions, n, out_ids, out_scores);
  return hipGetLastError();
}

hipError_t launch_zero_u32(uint32_t *p, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(64), 0, s, p, n);
  return hipGetLastError();
}

hipError_t launch_add_bf16(const uint16_t *a, const uint16_t *b, int64_t n, uint16_t *out, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(add_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, b, n, out);
  return hipGetLastError();
}

hipError_t launch_selftest_bf16(unsigned long long *count, hipStream_t s) {
  hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(1), 0, s, count);
  // 2^32 patterns: 2^14 blocks x 256 threads x 1024
  static_assert(16384ull * 256 * kSelfTestPerThread == (1ull << 32), "one pass over every pattern");
  hipLaunchKernelGGL(selftest_bf16_kernel, dim3(16384), dim3(256), 0, s, count);
  return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t *g, const uint16_t *u, int64_t n, uint16_t *out,
                         hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, n, out);
  return hipGetLastError();
}

hipError_t launch_combine(const uint16_t *rows, const uint32_t *inverse_order,
                          const uint16_t *scores, int T, int k, int D, int sorted,
                          const uint16_t *shared_out, const uint16_t *gate_logits,
                          uint16_t *sparse_out, uint16_t *y, hipStream_t s) {
  if ((int64_t)T * ((D + 7) / 8) <= 0) return hipSuccess;
  if (sorted)
    launch_combine_s<true>(rows, inverse_order, scores, T, k, D, shared_out, gate_logits, sparse_out, y, s);
  else
    launch_combine_s<false>(rows, inverse_order, scores, T, k, D, shared_out, gate_logits, sparse_out, y, s);
  return hipGetLastError();
}

hipError_t launch_combine_shared(const uint16_t *sparse, const uint16_t *shared_out,
                                 const uint16_t *gate_logits, int T, int D, uint16_t *y,
                                 hipStream_t s) {
  const int64_t n = (int64_t)T * D;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(combine_shared_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     sparse, shared_out, gate_logits, T, D, y);
  return hipGetLastError();
}

hipError_t launch_qgemv_rows(const uint16_t *x, int T, int K, const uint32_t *w,
                             const uint16_t *sc, const uint16_t *bi, int N, int bits, int group,
                             uint16_t *out, hipStream_t s) {
  const int items = T * N;
  if (items <= 0) return hipSuccess;
  const dim3 grid((items + 3) / 4), block(256);
  if (bits == 8)
    hipLaunchKernelGGL(qgemv_rows_kernel<8>, grid, block, 0, s, x, T, K, w, sc, bi, N, group, out);
  else
    hipLaunchKernelGGL(qgemv_rows_kernel<4>, grid, block, 0, s, x, T, K, w, sc, bi, N, group, out);
  return hipGetLastError();
}

}  // namespace astro
