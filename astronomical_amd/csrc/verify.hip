// Multi-token affine QMV for target-verification windows:
//   y[m][n] = sum_k x[m][k] * (s[n][k/g] * q[n][k] + b[n][k/g]),   m < M <= 16 token rows,
// the projection qwen3_5_target_verification_quantized_linear computes for an MTP window
// (qwen3_5/model/target_verification_quantized_linear.rs:232-330), which must equal the
// repeated one-token quantized_matmul bit for bit (:333-356 and the reference's test of it).
//
// The M token rows are the A operand (one 16-row block) of v_mfma_f32_16x16x32_{bf16,f16}
// and 16 weight rows the B operand.  A 32-input step never crosses an affine group, so the
// MFMA runs on the exact codes and the affine terms are applied once per group:
//   sum_k x (s q + b) = s * sum_k x (MAG + q) + (b - MAG s) * sum_k x,
// where MAG + q is made by OR-ing the code into the mantissa of MAG (bf16 128 for 4/5-bit
// codes; f16 1024 for every width) and bf16 8-bit codes are converted exactly (MAG = 0).
// Weight codes stream row-contiguously (16 B per lane) into a per-wave LDS ring by
// global->LDS DMA.  The window's x (in fragment order), its per-group sums and the
// workgroup rows' scales and biases are staged in LDS once per window of 2048 inputs.
// Every sum runs in an order fixed by K and the group size, and MFMA rows are
// independent, so an output depends only on its own token row: any M gives the bits of M = 1.
#include "common.h"
#include "kernels.h"

namespace astro {

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int VQ_WAVES = 8;
constexpr int VQ_THREADS = 64 * VQ_WAVES;
constexpr int VQ_STAGES = 3;                // code ring depth, stages of 128 inputs
constexpr int VQ_KW = 2048;                 // inputs per x window
constexpr int VQ_STEPS = VQ_KW / 32;        // 32-input MFMA steps per window

__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// LDS position of 16-B piece p of tile row r inside a ring slot: rows are BITS pieces
// long; the XOR spreads the 16 rows of one fragment read over the banks (80-B rows of
// 5-bit codes already do).
template <int BITS>
__device__ __forceinline__ int vq_swz(int r) {
  return BITS == 4 ? ((r >> 2) & 3) : BITS == 8 ? ((r >> 1) & 7) : 0;
}

// B fragment of 32-input step s of a ring slot: lane (n = lane % 16, g = lane / 16) holds
// the 8 codes of inputs 8 g .. 8 g + 7 of tile row n as four element pairs.  4/5-bit:
// pairs (j, j + 4) as MAG + q; 8-bit: pairs (2 j, 2 j + 1).
template <int BITS, bool F16>
__device__ __forceinline__ u32x4 vq_bfrag(const char *slot, int s, int lane) {
  const int n = lane & 15, g = lane >> 4;
  constexpr uint32_t M2 = F16 ? 0x64006400u : 0x43004300u;
  u32x4 o;
  if constexpr (BITS == 4) {
    const uint32_t wd = *(const uint32_t *)(slot + 16 * (n * 4 + (s ^ vq_swz<4>(n))) + 4 * g);
    o[0] = (wd & 0x000f000fu) | M2;
    o[1] = ((wd >> 4) & 0x000f000fu) | M2;
    o[2] = ((wd >> 8) & 0x000f000fu) | M2;
    o[3] = ((wd >> 12) & 0x000f000fu) | M2;
  } else if constexpr (BITS == 5) {
    // the 40 bits of the lane's 8 codes start at bit 8 g of word 5 s + g of the row
    const uint32_t *rw = (const uint32_t *)(slot + 80 * n) + 5 * s + g;
    const uint32_t wa = rw[0], wb = rw[1];
    const uint32_t lo = __builtin_amdgcn_alignbit(wb, wa, 8 * g), hi = wb >> (8 * g);
    o[0] = (lo & 0x1fu) | ((lo >> 4) & 0x1f0000u) | M2;
    o[1] = ((lo >> 5) & 0x1fu) | ((lo >> 9) & 0x1f0000u) | M2;
    o[2] = ((lo >> 10) & 0x1fu) | ((__builtin_amdgcn_alignbit(hi, lo, 30) & 0x1fu) << 16) | M2;
    o[3] = ((lo >> 15) & 0x1fu) | ((hi << 13) & 0x1f0000u) | M2;
  } else {
    const int p = 2 * s + (g >> 1);
    const uint2 ww = *(const uint2 *)(slot + 16 * (n * 8 + (p ^ vq_swz<8>(n))) + 8 * (g & 1));
    const uint32_t w2[2] = {ww.x, ww.y};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t v = w2[h];
      if constexpr (F16) {
        o[2 * h] = (v & 0xffu) | ((v & 0xff00u) << 8) | M2;
        o[2 * h + 1] = ((v >> 16) & 0xffu) | ((v >> 8) & 0xff0000u) | M2;
      } else {
        bf16x2 a, b;
        a[0] = (__bf16)(float)(v & 255u);
        a[1] = (__bf16)(float)((v >> 8) & 255u);
        b[0] = (__bf16)(float)((v >> 16) & 255u);
        b[1] = (__bf16)(float)(v >> 24);
        o[2 * h] = __builtin_bit_cast(uint32_t, a);
        o[2 * h + 1] = __builtin_bit_cast(uint32_t, b);
      }
    }
  }
  return o;
}

template <bool F16>
__device__ __forceinline__ f32x4 vq_mfma(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
}

// s_waitcnt vmcnt(n) for a compile-time n (expcnt and lgkmcnt not waited on)
template <int N>
__device__ __forceinline__ void vq_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
  asm volatile("" ::: "memory");
}

// LDS: [ring: waves x stages x 16 BITS pieces of 16 B][x fragments][group sums][scale|bias]
template <int BITS, int MR>
constexpr int vq_fixed_lds() {
  return VQ_WAVES * VQ_STAGES * 256 * BITS + VQ_STEPS * 4 * MR * 16 + VQ_STEPS * MR * 4;
}

template <int BITS, bool F16, int MR>
__global__ __launch_bounds__(VQ_THREADS) void vqmv_kernel(const uint16_t *__restrict__ x, int M, int K,
                                                          const uint32_t *__restrict__ w,
                                                          const uint16_t *__restrict__ sc,
                                                          const uint16_t *__restrict__ bi, int N, int group,
                                                          uint16_t *__restrict__ y) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  constexpr int PIECES = 16 * BITS;                  // 16-B pieces of a tile's stage
  constexpr int SLOT = 16 * PIECES;
  constexpr int NI = (PIECES + 63) / 64;             // DMA instructions per stage
  constexpr float MAG = F16 ? 1024.f : (BITS == 8 ? 0.f : 128.f);
  char *ring = lds;
  char *xa = ring + VQ_WAVES * VQ_STAGES * SLOT;
  float *xs = (float *)(xa + VQ_STEPS * 4 * MR * 16);
  uint32_t *sbl = (uint32_t *)(xs + VQ_STEPS * MR);
  float *xp = (float *)ring;  // 8-input partial sums of x while a window is staged

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows_blk = VQ_WAVES * 16;
  const int row0 = blockIdx.x * rows_blk;
  const int tile0 = row0 + wave * 16;
  const int64_t row_bytes = (int64_t)K * BITS / 8;
  const int gpr = K / group, spg = group / 32, lspg = __builtin_ctz((unsigned)spg);

  // DMA source of LDS position P = 64 i + lane: tile row P / BITS, piece (P % BITS) ^ swz
  const char *src[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    int P = 64 * i + lane;
    if (P >= PIECES) P = PIECES - 1;
    const int r = P / BITS, p = (P % BITS) ^ vq_swz<BITS>(r);
    const int n = tile0 + r < N ? tile0 + r : N - 1;  // rows past N load a valid row; never stored
    src[i] = (const char *)w + (int64_t)n * row_bytes + 16 * p;
  }
  char *myring = ring + wave * VQ_STAGES * SLOT;

  f32x4 yacc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += VQ_KW) {
    const int kw = K - k0 < VQ_KW ? K - k0 : VQ_KW;  // a multiple of 128
    const int nsteps = kw / 32, ngrp = kw / group, nstage = kw / 128;
    if (k0) __syncthreads();  // the previous window's LDS is consumed and every ring drained
    // x in fragment order (position (st, g, m)) and its 8-input partial sums
    for (int it = tid; it < nsteps * 4 * MR; it += VQ_THREADS) {
      const int st = it / (4 * MR), rem = it - st * 4 * MR, g = rem / MR, m = rem - g * MR;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M) v = *(const u32x4 *)(x + (int64_t)m * K + k0 + st * 32 + g * 8);
      float f[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[2 * j] = F16 ? h2f(v[j] & 0xffffu) : bf_lo(v[j]);
        f[2 * j + 1] = F16 ? h2f(v[j] >> 16) : bf_hi(v[j]);
      }
      u32x4 a = v;
      if (BITS != 8) {  // element pairs (j, j + 4), as the codes are paired
        a[0] = (v[0] & 0xffffu) | (v[2] << 16);
        a[1] = (v[0] >> 16) | (v[2] & 0xffff0000u);
        a[2] = (v[1] & 0xffffu) | (v[3] << 16);
        a[3] = (v[1] >> 16) | (v[3] & 0xffff0000u);
      }
      *(u32x4 *)(xa + it * 16) = a;
      xp[(st * 4 + g) * MR + m] = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
    }
    // the scale and bias of every (row, group) of the workgroup in this window
    for (int it = tid; it < rows_blk * ngrp; it += VQ_THREADS) {
      const int r = it / ngrp, gi = it - r * ngrp;
      const int n = row0 + r < N ? row0 + r : N - 1;
      const int64_t o = (int64_t)n * gpr + k0 / group + gi;
      sbl[it] = (uint32_t)sc[o] | ((uint32_t)bi[o] << 16);
    }
    __syncthreads();
    for (int it = tid; it < ngrp * MR; it += VQ_THREADS) {  // group sums, partials in input order
      const int gi = it / MR, m = it - gi * MR, per = group / 8;
      float s = 0.f;
      for (int j = 0; j < per; ++j) s += xp[(gi * per + j) * MR + m];
      xs[it] = s;
    }
    __syncthreads();  // xp (in the ring) is no longer read

    const int64_t stage0 = (int64_t)(k0 / 128) * 16 * BITS;  // window start within a row
    auto issue = [&](int j) {  // stage j (clamped to the window's last) into its ring slot
      const int jj = j < nstage ? j : nstage - 1;
      char *slot = myring + (j % VQ_STAGES) * SLOT;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        if (i + 1 < NI || PIECES % 64 == 0 || lane < PIECES - 64 * (NI - 1))
          __builtin_amdgcn_global_load_lds((const void *)(src[i] + stage0 + (int64_t)jj * 16 * BITS),
                                           (lds_void *)(slot + i * 1024), 16, 0, 0);
      }
    };
#pragma unroll
    for (int j = 0; j < VQ_STAGES - 1; ++j) issue(j);
    const int m_lane = lane & 15, g_lane = lane >> 4;
    const int rl = wave * 16 + m_lane;  // this lane's B row within the workgroup
    f32x4 gacc = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < nstage; ++j) {
      vq_wait_vmcnt<NI * (VQ_STAGES - 2)>();  // this wave's stage j is in LDS
      issue(j + VQ_STAGES - 1);               // into the slot consumed at j - 1
      const char *slot = myring + (j % VQ_STAGES) * SLOT;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int st = 4 * j + s;
        const u32x4 av = *(const u32x4 *)(xa + ((st * 4 + g_lane) * MR + (m_lane % MR)) * 16);
        const u32x4 bv = vq_bfrag<BITS, F16>(slot, s, lane);
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        gacc = vq_mfma<F16>(av, bv, (s & (spg - 1)) == 0 ? zero : gacc);
        if ((s & (spg - 1)) == spg - 1) {  // last step of group gi: apply its affine terms
          const int gi = st >> lspg;
          const f32x4 xsv = *(const f32x4 *)(xs + gi * MR + ((4 * g_lane) % MR));
          const uint32_t sb = sbl[rl * ngrp + gi];
          const float sv = F16 ? h2f(sb & 0xffffu) : bf_lo(sb);
          const float bv2 = F16 ? h2f(sb >> 16) : bf_hi(sb);
          const float bp = __builtin_fmaf(-MAG, sv, bv2);
#pragma unroll
          for (int i = 0; i < 4; ++i) yacc[i] = __builtin_fmaf(sv, gacc[i], __builtin_fmaf(bp, xsv[i], yacc[i]));
        }
      }
    }
    vq_wait_vmcnt<0>();  // the clamped trailing stages
  }
  // lane holds tokens 4 g + i of tile row m_lane
  const int n = tile0 + (lane & 15);
  if (n >= N) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * (lane >> 4) + i;
    if (m < M) y[(int64_t)m * N + n] = (uint16_t)(F16 ? f2h(yacc[i]) : f2bf(yacc[i]));
  }
}

template <int BITS, bool F16, int MR>
hipError_t launch_vq(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc, const uint16_t *bi,
                     int N, int group, uint16_t *y, hipStream_t s) {
  const int kw = K < VQ_KW ? K : VQ_KW;
  const int lds = vq_fixed_lds<BITS, MR>() + VQ_WAVES * 16 * (kw / group) * 4;
  static bool raised = false;  // > 64 KB of LDS is an opt-in per kernel: the largest (group 32)
  auto kern = vqmv_kernel<BITS, F16, MR>;
  if (!raised) {
    const int most = vq_fixed_lds<BITS, MR>() + VQ_WAVES * 16 * (VQ_KW / 32) * 4;
    const hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, most);
    if (e != hipSuccess) return e;
    raised = true;
  }
  const int rows_blk = VQ_WAVES * 16;
  hipLaunchKernelGGL(kern, dim3((unsigned)((N + rows_blk - 1) / rows_blk)), dim3(VQ_THREADS), lds, s, x, M, K, w,
                     sc, bi, N, group, y);
  return hipGetLastError();
}

template <int BITS, bool F16>
hipError_t launch_vq_m(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc, const uint16_t *bi,
                       int N, int group, uint16_t *y, hipStream_t s) {
  if (M <= 8) return launch_vq<BITS, F16, 8>(x, M, K, w, sc, bi, N, group, y, s);
  return launch_vq<BITS, F16, 16>(x, M, K, w, sc, bi, N, group, y, s);
}

}  // namespace

bool verify_qmv_supported(int K, int bits, int group, const void *x, const void *w) {
  return (bits == 4 || bits == 5 || bits == 8) && (group == 32 || group == 64 || group == 128) && K > 0 &&
         K % 128 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0;
}

hipError_t launch_verify_qmv(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc,
                             const uint16_t *bi, int N, int bits, int group, bool f16, uint16_t *y, hipStream_t s) {
  for (int m0 = 0; m0 < M; m0 += kVerifyRows) {  // one 16-row MFMA block per launch
    const int mm = M - m0 < kVerifyRows ? M - m0 : kVerifyRows;
    const uint16_t *xm = x + (int64_t)m0 * K;
    uint16_t *ym = y + (int64_t)m0 * N;
    hipError_t e;
    if (bits == 4)
      e = f16 ? launch_vq_m<4, true>(xm, mm, K, w, sc, bi, N, group, ym, s)
              : launch_vq_m<4, false>(xm, mm, K, w, sc, bi, N, group, ym, s);
    else if (bits == 5)
      e = f16 ? launch_vq_m<5, true>(xm, mm, K, w, sc, bi, N, group, ym, s)
              : launch_vq_m<5, false>(xm, mm, K, w, sc, bi, N, group, ym, s);
    else
      e = f16 ? launch_vq_m<8, true>(xm, mm, K, w, sc, bi, N, group, ym, s)
              : launch_vq_m<8, false>(xm, mm, K, w, sc, bi, N, group, ym, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace astro
