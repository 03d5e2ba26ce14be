// Bandwidth-bound pieces of the block: SwiGLU, the weighted expert combine with the
// shared expert's gated add, and a skinny quantized GEMV (the shared expert's
// 2048 -> 1 output gate).
#include "common.h"
#include "kernels.h"

namespace astro {

namespace {

constexpr int kHoistK = 16;  // top-k widths whose combine loads are all issued up front

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *__restrict__ g,
                                                     const uint16_t *__restrict__ u, int64_t n,
                                                     uint16_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (uint16_t)swiglu_bf(bf2f(g[i]), bf2f(u[i]));
}

// y[t][d] for 8 consecutive d per thread.  Row of assignment (t, j): inverse_order[t*k+j]
// (or t*k+j when inverse_order is null).  sorted: fp32 fma accumulation of out*score in
// slot order, one bf16 rounding (weighted_sum.rs:16-33).  unsorted: bf16 product per
// slot, fp32 accumulation, one bf16 rounding (weighted_sum.rs:112-119).  Then, with a
// shared expert: y = bf16(sparse + bf16(shared * bf16(sigmoid(z)))) (output_combination.rs:40-42).
template <bool VEC>
__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t *__restrict__ rows, const uint32_t *__restrict__ inverse_order,
    const uint16_t *__restrict__ scores, int T, int k, int D, int sorted,
    const uint16_t *__restrict__ shared_out, const uint16_t *__restrict__ gate_logits,
    uint16_t *__restrict__ sparse_out, uint16_t *__restrict__ y) {
#pragma clang fp contract(off)
  const int chunks = (D + 7) >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)T * chunks) return;
  const int t = (int)(gid / chunks), d0 = (int)(gid % chunks) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (VEC && k >= 1 && k <= kHoistK) {
    // every index, score and row load is issued before the first use; slots past k
    // repeat the last slot and are masked out of the (ordered) accumulation
    uint32_t inv[kHoistK];
    float sc[kHoistK];
#pragma unroll
    for (int j = 0; j < kHoistK; ++j) {
      const int64_t a = (int64_t)t * k + (j < k ? j : k - 1);
      inv[j] = inverse_order ? inverse_order[a] : (uint32_t)a;
      sc[j] = bf2f(scores[a]);
    }
    u32x4 q[kHoistK];
#pragma unroll
    for (int j = 0; j < kHoistK; ++j) q[j] = *(const u32x4 *)(rows + (int64_t)inv[j] * D + d0);
#pragma unroll
    for (int j = 0; j < kHoistK; ++j) {
      const bool on = j < k;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = (i & 1) ? bf_hi(q[j][i >> 1]) : bf_lo(q[j][i >> 1]);
        const float nxt = sorted ? __builtin_fmaf(v, sc[j], acc[i]) : acc[i] + round_bf(v * sc[j]);
        acc[i] = on ? nxt : acc[i];
      }
    }
  } else
  for (int j = 0; j < k; ++j) {
    const int64_t a = (int64_t)t * k + j;
    const int64_t r = inverse_order ? (int64_t)inverse_order[a] : a;
    const float s = bf2f(scores[a]);
    const uint16_t *src = rows + r * D + d0;
    float v[8];
    if (VEC) {
      const u32x4 q = *(const u32x4 *)src;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf_lo(q[i]);
        v[2 * i + 1] = bf_hi(q[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = d0 + i < D ? bf2f(src[i]) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (sorted) acc[i] = __builtin_fmaf(v[i], s, acc[i]);
      else acc[i] = acc[i] + round_bf(v[i] * s);
    }
  }
  uint32_t outb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) outb[i] = f2bf(acc[i]);
  if (sparse_out) {
    uint16_t *dst = sparse_out + (int64_t)t * D + d0;
    for (int i = 0; i < 8; ++i)
      if (d0 + i < D) dst[i] = (uint16_t)outb[i];
  }
  if (shared_out) {
    const float gate = round_bf(det_sigmoid(bf2f(gate_logits[t])));
    const uint16_t *so = shared_out + (int64_t)t * D + d0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float sv = (VEC || d0 + i < D) ? bf2f(so[i]) : 0.f;
      outb[i] = f2bf(bf2f(outb[i]) + round_bf(sv * gate));
    }
  }
  uint16_t *dst = y + (int64_t)t * D + d0;
  if (VEC) {
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

// One wave per (token, output row): lane l covers inputs 32l.. of each 2048-wide chunk,
// dequantising in fp32 (scale*q + bias) and accumulating x*w with fma; wave tree sum.
template <int BITS>
__global__ __launch_bounds__(256) void qgemv_rows_kernel(
    const uint16_t *__restrict__ x, int T, int K, const uint32_t *__restrict__ w,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ bi, int N, int group,
    uint16_t *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= T * N) return;
  const int t = item / N, n = item % N;
  const int wpr = K * BITS / 32;          // words per row
  const uint32_t *wr = w + (int64_t)n * wpr;
  const uint16_t *sr = sc + (int64_t)n * (K / group);
  const uint16_t *br = bi + (int64_t)n * (K / group);
  const uint16_t *xr = x + (int64_t)t * K;
  float acc = 0.f;
  for (int k0 = lane * 32; k0 < K; k0 += 64 * 32) {
    const float s = bf2f(sr[k0 / group]), b = bf2f(br[k0 / group]);
    const u32x4 *xp = (const u32x4 *)(xr + k0);
    float xv[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 q = xp[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[8 * c + 2 * i] = bf_lo(q[i]);
        xv[8 * c + 2 * i + 1] = bf_hi(q[i]);
      }
    }
    const uint32_t *wp = wr + k0 * BITS / 32;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t word = wp[i * BITS / 32];
      const float q = (float)((word >> ((i * BITS) & 31)) & ((1u << BITS) - 1u));
      acc = __builtin_fmaf(xv[i], __builtin_fmaf(s, q, b), acc);
    }
  }
  acc = wave_sum_fast(acc);
  if (lane == 0) out[(int64_t)t * N + n] = (uint16_t)f2bf(acc);
}

}  // namespace

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
  const int64_t threads = (int64_t)T * ((D + 7) / 8);
  if (threads <= 0) return hipSuccess;
  const dim3 grid((unsigned)((threads + 255) / 256));
  const bool vec = (D % 8) == 0 && ((uintptr_t)rows % 16) == 0 && ((uintptr_t)y % 16) == 0;
  if (vec)
    hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, s, rows, inverse_order, scores,
                       T, k, D, sorted, shared_out, gate_logits, sparse_out, y);
  else
    hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, s, rows, inverse_order, scores,
                       T, k, D, sorted, shared_out, gate_logits, sparse_out, y);
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
