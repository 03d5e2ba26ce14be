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

#include <algorithm>

namespace astro {

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));


__device__ __forceinline__ float h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// LDS position of 16-B piece p of tile row r inside a ring slot: rows are PPR pieces long;
// the XOR spreads the 16 rows of one fragment read over the banks (80-B rows of 5-bit codes
// already do).
template <int PPR>
__device__ __forceinline__ int vq_swz(int r) {
  return PPR == 4 ? ((r >> 2) & 3) : PPR == 8 ? ((r >> 1) & 7) : 0;
}

// Codes of 32-input step s of a ring slot for lane (n = lane % 16, g = lane / 16): the 8
// codes of inputs 8 g .. 8 g + 7 of tile row n (4-bit: one word; 5-bit: the two words holding
// their 40 bits, which start at bit 8 g of the first; 8-bit: two words).
template <int BITS, int PPR>
__device__ __forceinline__ uint2 vq_braw(const char *slot, int s, int lane) {
  const int n = lane & 15, g = lane >> 4;
  if constexpr (BITS == 4) {
    return make_uint2(*(const uint32_t *)(slot + 16 * (n * PPR + (s ^ vq_swz<PPR>(n))) + 4 * g), 0u);
  } else if constexpr (BITS == 5) {
    const uint32_t *rw = (const uint32_t *)(slot + 16 * PPR * n) + 5 * s + g;
    return make_uint2(rw[0], rw[1]);
  } else {
    const int p = 2 * s + (g >> 1);
    return *(const uint2 *)(slot + 16 * (n * PPR + (p ^ vq_swz<PPR>(n))) + 8 * (g & 1));
  }
}

// The B fragment from those codes: four element pairs, (j, j + 4) as MAG + q for 4/5-bit
// codes, (2 j, 2 j + 1) for 8-bit codes.
template <int BITS, bool F16>
__device__ __forceinline__ u32x4 vq_bconv(uint2 raw, int lane) {
  constexpr uint32_t M2 = F16 ? 0x64006400u : 0x43004300u;
  u32x4 o;
  if constexpr (BITS == 4) {
    const uint32_t wd = raw.x;
    o[0] = (wd & 0x000f000fu) | M2;
    o[1] = ((wd >> 4) & 0x000f000fu) | M2;
    o[2] = ((wd >> 8) & 0x000f000fu) | M2;
    o[3] = ((wd >> 12) & 0x000f000fu) | M2;
  } else if constexpr (BITS == 5) {
    const int g = lane >> 4;
    const uint32_t lo = __builtin_amdgcn_alignbit(raw.y, raw.x, 8 * g), hi = raw.y >> (8 * g);
    o[0] = (lo & 0x1fu) | ((lo >> 4) & 0x1f0000u) | M2;
    o[1] = ((lo >> 5) & 0x1fu) | ((lo >> 9) & 0x1f0000u) | M2;
    o[2] = ((lo >> 10) & 0x1fu) | ((__builtin_amdgcn_alignbit(hi, lo, 30) & 0x1fu) << 16) | M2;
    o[3] = ((lo >> 15) & 0x1fu) | ((hi << 13) & 0x1f0000u) | M2;
  } else {
    const uint32_t w2[2] = {raw.x, raw.y};
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

// inputs per x window: 2048, or 1024 for 32-input groups (their scales take twice the room)
template <int G>
constexpr int vq_window() {
  return G == 32 ? 1024 : 2048;
}

// LDS: [ring: waves x stages x 16 rows x SPS * BITS / 4 pieces of 16 B][x fragments]
// [group sums][scale | bias]
template <int BITS, int MR, int G, int SPS, int NS, int W>
constexpr int vq_lds_bytes() {
  constexpr int KW = vq_window<G>();
  return W * NS * 64 * SPS * BITS + (KW / 32) * 4 * MR * 16 + (KW / G) * MR * 4 + W * 16 * (KW / G) * 4;
}

// 4 waves per SIMD: two resident workgroups per CU (128 VGPRs)
// SPS: 32-input steps per ring stage (8: runs of 128 B or more of each row per stage); NS:
// ring stages (NS - 1 in flight); W: waves per workgroup (16 W rows per tile)
template <int BITS, bool F16, int MR, int G, int SPS, int NS, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(4))) void vqmv_kernel(const uint16_t *__restrict__ x, int M, int K,
                                                          const uint32_t *__restrict__ w,
                                                          const uint16_t *__restrict__ sc,
                                                          const uint16_t *__restrict__ bi, int N,
                                                          uint16_t *__restrict__ y) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  constexpr int PPR = SPS * BITS / 4;                // 16-B pieces of a row's stage
  constexpr int SIN = 32 * SPS;                      // inputs per stage
  constexpr int PIECES = 16 * PPR;                   // 16-B pieces of a tile's stage
  constexpr int SLOT = 16 * PIECES;
  constexpr int NI = (PIECES + 63) / 64;             // DMA instructions per stage
  constexpr int KW = vq_window<G>(), GW = KW / G;    // window inputs and groups
  constexpr int SPG = G / 32;                        // steps per group
  constexpr float MAG = F16 ? 1024.f : (BITS == 8 ? 0.f : 128.f);
  char *ring = lds;
  char *xa = ring + W * NS * SLOT;
  float *xs = (float *)(xa + (KW / 32) * 4 * MR * 16);  // [group][token]
  uint32_t *sbl = (uint32_t *)(xs + GW * MR);           // [row of the workgroup][group]: s | b << 16

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t row_bytes = (int64_t)K * BITS / 8;
  const int gpr = K / G;
  const int nwin = (K + KW - 1) / KW;
  // workgroup tiles of 128 rows, this workgroup's are blockIdx.x + k gridDim.x
  const int ntiles = (N + W * 16 - 1) / (W * 16);
  const int nk = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int nstage_all = K / SIN;  // stages of one tile
  auto tile_row = [&](int k) { return ((int)blockIdx.x + k * (int)gridDim.x) * (W * 16) + wave * 16; };

  // DMA of LDS position P = 64 i + lane: tile row P / BITS, piece (P % BITS) ^ swz
  int dma_r[NI], dma_off[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    int P = 64 * i + lane;
    if (P >= PIECES) P = PIECES - 1;
    dma_r[i] = P / PPR;
    dma_off[i] = 16 * ((P % PPR) ^ vq_swz<PPR>(dma_r[i]));
  }
  char *myring = ring + wave * NS * SLOT;
  auto issue = [&](int q) {  // stage q of this workgroup's (tile, stage) sequence, clamped to the last
    const int last = nk * nstage_all - 1;
    const int qq = q < last ? q : last;
    const int k = qq / nstage_all, st = qq - k * nstage_all;
    const int t0 = tile_row(k);
    char *slot = myring + (q % NS) * SLOT;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int n = t0 + dma_r[i] < N ? t0 + dma_r[i] : N - 1;  // rows past N load a valid row; never stored
      if (i + 1 < NI || PIECES % 64 == 0 || lane < PIECES - 64 * (NI - 1))
        __builtin_amdgcn_global_load_lds(
            (const void *)((const char *)w + (int64_t)n * row_bytes + dma_off[i] + (int64_t)st * 16 * PPR),
            (lds_void *)(slot + i * 1024), 16, 0, 0);
    }
  };
  // the first stages stream while x and the affine terms are staged
#pragma unroll
  for (int q = 0; q < NS - 1; ++q) issue(q);

  // this wave's rows' scale | bias of window k0 of tile row t0 (16-B pieces of 8 groups when
  // rows and bases allow; each lane then holds at most one piece of each)
  const bool vec_sb = gpr % 8 == 0 && ((uintptr_t)sc % 16) == 0 && ((uintptr_t)bi % 16) == 0;
  auto sb_piece = [&](int t0, int k0, int ngrp, u32x4 &sv, u32x4 &bv) {
    const int pr = ngrp / 8, r = lane / pr, pc = lane - r * pr;
    const int n = t0 + r < N ? t0 + r : N - 1;
    const int64_t o = (int64_t)n * gpr + k0 / G + 8 * pc;
    sv = *(const u32x4 *)(sc + o);
    bv = *(const u32x4 *)(bi + o);
  };
  auto sb_store = [&](int ngrp, const u32x4 &sv, const u32x4 &bv) {
    const int pr = ngrp / 8, r = lane / pr, pc = lane - r * pr;
    u32x4 lo, hi;  // (s, b) of groups 8 pc + 0..3 and 8 pc + 4..7
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      lo[2 * q] = (sv[q] & 0xffffu) | (bv[q] << 16);
      lo[2 * q + 1] = (sv[q] >> 16) | (bv[q] & 0xffff0000u);
      hi[2 * q] = (sv[q + 2] & 0xffffu) | (bv[q + 2] << 16);
      hi[2 * q + 1] = (sv[q + 2] >> 16) | (bv[q + 2] & 0xffff0000u);
    }
    uint32_t *d = sbl + (wave * 16 + r) * GW + 8 * pc;
    *(u32x4 *)d = lo;
    *(u32x4 *)(d + 4) = hi;
  };
  auto sb_load = [&](int t0, int k0, int ngrp) {
    if (vec_sb && ngrp % 8 == 0) {
      if (lane < 16 * (ngrp / 8)) {
        u32x4 sv, bv;
        sb_piece(t0, k0, ngrp, sv, bv);
        sb_store(ngrp, sv, bv);
      }
    } else {
      for (int it = lane; it < 16 * ngrp; it += 64) {
        const int r = it / ngrp, gi = it - r * ngrp;
        const int n = t0 + r < N ? t0 + r : N - 1;
        const int64_t o = (int64_t)n * gpr + k0 / G + gi;
        sbl[(wave * 16 + r) * GW + gi] = (uint32_t)sc[o] | ((uint32_t)bi[o] << 16);
      }
    }
  };
  // one window per tile and one piece per lane: the next tile's terms are fetched during
  // this tile and written to LDS at the tile boundary
  const bool prefetch = nwin == 1 && vec_sb && gpr % 8 == 0 && 16 * (gpr / 8) <= 64;
  const int pref_at = nstage_all > NS ? nstage_all - NS : 0;
  u32x4 pf_s = {0u, 0u, 0u, 0u}, pf_b = {0u, 0u, 0u, 0u};

  const int m_lane = lane & 15, g_lane = lane >> 4;
  const int rl = wave * 16 + m_lane;  // this lane's B row within the workgroup
  f32x4 yacc = {0.f, 0.f, 0.f, 0.f}, ydone = {0.f, 0.f, 0.f, 0.f};
  int done_row = -1;  // tile row of ydone, stored after the next DMA issue
  auto store = [&](int t0, const f32x4 &v) {
    const int n = t0 + m_lane;
    if (n >= N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * g_lane + i;
      if (m < M) y[(int64_t)m * N + n] = (uint16_t)(F16 ? f2h(v[i]) : f2bf(v[i]));
    }
  };
  int q = 0;  // (tile, stage) sequence number
  for (int k = 0; k < nk; ++k) {
    const int t0 = tile_row(k);
    for (int k0 = 0; k0 < K; k0 += KW) {
      const int kw = K - k0 < KW ? K - k0 : KW;  // a multiple of 128
      const int ngrp = kw / G, nstage = kw / SIN;
      const bool stage_x = nwin > 1 || k == 0;
      if (stage_x) {
        if (k || k0) __syncthreads();  // every wave is done with the previous window
        // x in fragment order (position (step, g, m)) and its group sums, one (group, token)
        // per thread: 8-input partial sums added in input order
        for (int it = tid; it < ngrp * MR; it += 64 * W) {
          const int gi = it / MR, m = it % MR;
          float sum = 0.f;
          constexpr int CB = G / 8 < 8 ? G / 8 : 8;  // chunks loaded together
#pragma unroll 1
          for (int c0 = 0; c0 < G / 8; c0 += CB) {
            u32x4 vb[CB];
#pragma unroll
            for (int c = 0; c < CB; ++c) {
              vb[c] = u32x4{0u, 0u, 0u, 0u};
              if (m < M) vb[c] = *(const u32x4 *)(x + (int64_t)m * K + k0 + gi * G + 8 * (c0 + c));
            }
#pragma unroll
            for (int c = 0; c < CB; ++c) {
              const int kk = gi * G + 8 * (c0 + c);
              const u32x4 v = vb[c];
              float f[8];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                f[2 * e] = F16 ? h2f(v[e] & 0xffffu) : bf_lo(v[e]);
                f[2 * e + 1] = F16 ? h2f(v[e] >> 16) : bf_hi(v[e]);
              }
              sum += ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
              u32x4 a = v;
              if (BITS != 8) {  // element pairs (j, j + 4), as the codes are paired
                a[0] = (v[0] & 0xffffu) | (v[2] << 16);
                a[1] = (v[0] >> 16) | (v[2] & 0xffff0000u);
                a[2] = (v[1] & 0xffffu) | (v[3] << 16);
                a[3] = (v[1] >> 16) | (v[3] & 0xffff0000u);
              }
              *(u32x4 *)(xa + (((kk >> 5) * 4 + ((kk >> 3) & 3)) * MR + m) * 16) = a;
            }
          }
          xs[gi * MR + m] = sum;
        }
      }
      if (prefetch && k > 0) {
        if (lane < 16 * (ngrp / 8)) sb_store(ngrp, pf_s, pf_b);
      } else {
        sb_load(t0, k0, ngrp);
      }
      if (stage_x) __syncthreads();  // x fragments and sums are in LDS

      for (int jw = 0; jw < nstage; ++jw, ++q) {
        vq_wait_vmcnt<NI * (NS - 2)>();  // this wave's stage q is in LDS
        if (done_row >= 0) {  // the previous tile's outputs, behind its last wait
          store(done_row, ydone);
          done_row = -1;
        }
        if (prefetch && jw == pref_at && k + 1 < nk && lane < 16 * (ngrp / 8)) {
          // the next tile's scale and bias pieces.  Plain asm loads: the compiler does not
          // track them, and this wave's vmcnt waits of the following stages (which leave
          // only the newer DMA stages outstanding) cover them before the tile boundary
          const int pr = ngrp / 8, r = lane / pr, pc = lane - r * pr;
          const int t1 = tile_row(k + 1), n = t1 + r < N ? t1 + r : N - 1;
          const int64_t o = (int64_t)n * gpr + 8 * pc;
          asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(pf_s) : "v"(sc + o) : "memory");
          asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(pf_b) : "v"(bi + o) : "memory");
        }
        issue(q + NS - 1);  // into the slot consumed at q - 1
        const char *slot = myring + (q % NS) * SLOT;
        // the stage in halves of 4 steps, each a whole number of groups: every LDS read of a
        // half first, one accumulator per group (independent MFMA chains), then the affine
        // terms of its groups in input order
        constexpr int HG = 4 / SPG;  // groups per half
#pragma unroll
        for (int h = 0; h < SPS / 4; ++h) {
          u32x4 av[4];
          uint2 raw[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int st = SPS * jw + 4 * h + s;
            av[s] = *(const u32x4 *)(xa + ((st * 4 + g_lane) * MR + (m_lane % MR)) * 16);
            raw[s] = vq_braw<BITS, PPR>(slot, 4 * h + s, lane);
          }
          uint32_t sbv[HG];
          f32x4 xsv[HG];
#pragma unroll
          for (int e = 0; e < HG; ++e) {
            const int gi = (SPS * jw + 4 * h) / SPG + e;
            sbv[e] = sbl[rl * GW + gi];
            xsv[e] = *(const f32x4 *)(xs + gi * MR + ((4 * g_lane) % MR));
          }
          f32x4 acc[HG];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int e = s / SPG;
            const u32x4 bv = vq_bconv<BITS, F16>(raw[s], lane);
            if (s % SPG == 0) {
              const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
              acc[e] = vq_mfma<F16>(av[s], bv, zero);
            } else {
              acc[e] = vq_mfma<F16>(av[s], bv, acc[e]);
            }
          }
#pragma unroll
          for (int e = 0; e < HG; ++e) {
            const float sv = F16 ? h2f(sbv[e] & 0xffffu) : bf_lo(sbv[e]);
            const float bv2 = F16 ? h2f(sbv[e] >> 16) : bf_hi(sbv[e]);
            const float bp = __builtin_fmaf(-MAG, sv, bv2);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              yacc[i] = __builtin_fmaf(sv, acc[e][i], __builtin_fmaf(bp, xsv[e][i], yacc[i]));
          }
        }
      }
    }
    ydone = yacc;  // lane holds tokens 4 g + i of tile row m_lane
    done_row = t0;
    yacc = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  vq_wait_vmcnt<0>();  // the clamped trailing stages
  if (done_row >= 0) store(done_row, ydone);
}

// compute units of the current device (cached per device)
int vq_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

template <int BITS, bool F16, int MR, int G, int SPS, int NS, int W = 8>
hipError_t launch_vq(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc, const uint16_t *bi,
                     int N, uint16_t *y, hipStream_t s) {
  constexpr int lds = vq_lds_bytes<BITS, MR, G, SPS, NS, W>();
  static bool raised = false;  // > 64 KB of LDS is an opt-in per kernel
  auto kern = vqmv_kernel<BITS, F16, MR, G, SPS, NS, W>;
  if (!raised) {
    const hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    raised = true;
  }
  // persistent workgroups: as many as are resident at once (LDS bound), each walks tiles
  const int rows_blk = W * 16, ntiles = (N + rows_blk - 1) / rows_blk;
  const int per_cu = (160 * 1024) / lds > 0 ? (160 * 1024) / lds : 1;
  const int grid = std::min(ntiles, vq_cus() * per_cu);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * W), lds, s, x, M, K, w, sc, bi, N, y);
  return hipGetLastError();
}

// Stage shape per window size (measured on the c1 logits head): 8-step stages (128-B or longer
// runs of each row) with two in the ring for up to 4 tokens, and for 5..8 tokens of 4-bit codes
// with 7-wave workgroups (two per CU still fit); three in the ring for 9..16 tokens (one
// workgroup per CU).
template <int BITS, bool F16, int MR, int G>
hipError_t launch_vq_s(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc, const uint16_t *bi,
                       int N, uint16_t *y, hipStream_t s) {
  constexpr bool wide_ok = BITS != 8;
  if (wide_ok && K % 256 == 0) {
    if (MR == 4) return launch_vq<BITS, F16, MR, G, 8, 2>(x, M, K, w, sc, bi, N, y, s);
    if (MR == 8 && BITS == 4) return launch_vq<BITS, F16, MR, G, 8, 2, 7>(x, M, K, w, sc, bi, N, y, s);
    if (MR == 16) return launch_vq<BITS, F16, MR, G, 8, 3>(x, M, K, w, sc, bi, N, y, s);
  }
  return launch_vq<BITS, F16, MR, G, 4, 3>(x, M, K, w, sc, bi, N, y, s);
}

template <int BITS, bool F16, int MR>
hipError_t launch_vq_g(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc, const uint16_t *bi,
                       int N, int group, uint16_t *y, hipStream_t s) {
  if (group == 32) return launch_vq_s<BITS, F16, MR, 32>(x, M, K, w, sc, bi, N, y, s);
  if (group == 64) return launch_vq_s<BITS, F16, MR, 64>(x, M, K, w, sc, bi, N, y, s);
  return launch_vq_s<BITS, F16, MR, 128>(x, M, K, w, sc, bi, N, y, s);
}

template <int BITS, bool F16>
hipError_t launch_vq_m(const uint16_t *x, int M, int K, const uint32_t *w, const uint16_t *sc, const uint16_t *bi,
                       int N, int group, uint16_t *y, hipStream_t s) {
  if (M <= 4) return launch_vq_g<BITS, F16, 4>(x, M, K, w, sc, bi, N, group, y, s);
  if (M <= 8) return launch_vq_g<BITS, F16, 8>(x, M, K, w, sc, bi, N, group, y, s);
  return launch_vq_g<BITS, F16, 16>(x, M, K, w, sc, bi, N, group, y, s);
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
