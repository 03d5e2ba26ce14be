// Grouped GEMM for the gathered expert projections (gather_qmm), the shared expert
// and the router: bf16 MFMA (v_mfma_f32_16x16x32_bf16) over tiles of up to 128 rows of
// one expert x 128 weight rows, K stepped by 64.
//
// Per K step a workgroup (4 waves) stages
//   - the activation tile: up to 128 rows gathered through the sort permutation
//     (row r of expert e reads x[sorted_order[r] / k]) -> LDS, 16 B per lane-load;
//   - the weight tile: 128 rows x 64 inputs of MLX affine codes (4-bit: 32 B, 8-bit:
//     64 B per row) loaded coalesced, dequantised in registers (scale*q + bias, fp32)
//     to bf16 and written to LDS; dense bf16 weights are copied as-is.
// Each wave owns 32 output columns (plain) or 16 activated columns = 16 gate + 16 up
// columns (SwiGLU epilogue) and every valid 16-row block of the tile; 16-row blocks
// beyond the expert's rows are skipped, so ragged experts cost at most 15 wasted rows.
// The next K step's global loads are issued before the MFMAs of the current one.
#include "common.h"
#include "gemm_dev.h"
#include "kernels.h"

#include <algorithm>
#include <type_traits>

namespace astro {

namespace {

constexpr int BR = 128;      // weight rows per tile
constexpr int BK = 64;       // K step
constexpr int LDSP = BK + 8; // padded LDS row (bf16 elements); 144 B keeps 16 B alignment

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf2_hw(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// Raw loads of one K step's weights: codes (or dense bf16) and the group's scale and bias as
// bf16 bits.  The bits are widened to float only when the step is dequantised, so nothing
// waits for these loads when they are issued.
struct BRegs {
  u32x4 q[4];
  uint32_t s, b;
};

template <int KIND>
__device__ __forceinline__ void load_b(BRegs &r, const uint32_t *wrow, const uint16_t *srow,
                                       const uint16_t *brow, const uint16_t *drow, int k0,
                                       int half, int group) {
  if (KIND == kBQ4) {
    r.q[0] = *(const u32x4 *)(wrow + (k0 >> 3) + half * 4);
    const int g = (k0 + 32 * half) / group;
    r.s = srow[g];
    r.b = brow[g];
  } else if (KIND == kBQ8) {
    const u32x4 *p = (const u32x4 *)(wrow + (k0 >> 2) + half * 8);
    r.q[0] = p[0];
    r.q[1] = p[1];
    const int g = (k0 + 32 * half) / group;
    r.s = srow[g];
    r.b = brow[g];
  } else {
    const u32x4 *p = (const u32x4 *)(drow + k0 + half * 32);
    r.q[0] = p[0];
    r.q[1] = p[1];
    r.q[2] = p[2];
    r.q[3] = p[3];
  }
}

// dequantise 32 codes (inputs 32*half .. +32 of the K step) into 16 bf16 pairs
template <int KIND>
__device__ __forceinline__ void store_b(uint16_t *dst, const BRegs &r, bool valid) {
  u32x4 out[4];
  if (!valid) {
    for (int i = 0; i < 4; ++i) out[i] = u32x4{0, 0, 0, 0};
  } else if (KIND == kBQ4) {
    const float sc = bf2f(r.s), bi = bf2f(r.b);
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
      const uint32_t w = r.q[0][wi];
      uint32_t p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float q0 = (float)((w >> (8 * j)) & 15u);
        const float q1 = (float)((w >> (8 * j + 4)) & 15u);
        p[j] = pack_bf2_hw(__builtin_fmaf(sc, q0, bi), __builtin_fmaf(sc, q1, bi));
      }
      out[wi] = u32x4{p[0], p[1], p[2], p[3]};
    }
  } else if (KIND == kBQ8) {
    const float sc = bf2f(r.s), bi = bf2f(r.b);
#pragma unroll
    for (int wi = 0; wi < 8; ++wi) {
      const uint32_t w = r.q[wi >> 2][wi & 3];
      const float q0 = (float)(w & 255u), q1 = (float)((w >> 8) & 255u);
      const float q2 = (float)((w >> 16) & 255u), q3 = (float)(w >> 24);
      const uint32_t p0 = pack_bf2_hw(__builtin_fmaf(sc, q0, bi), __builtin_fmaf(sc, q1, bi));
      const uint32_t p1 = pack_bf2_hw(__builtin_fmaf(sc, q2, bi), __builtin_fmaf(sc, q3, bi));
      out[wi >> 1][(wi & 1) * 2] = p0;
      out[wi >> 1][(wi & 1) * 2 + 1] = p1;
    }
  } else {
    for (int i = 0; i < 4; ++i) out[i] = r.q[i];
  }
  u32x4 *d = (u32x4 *)dst;
  d[0] = out[0];
  d[1] = out[1];
  d[2] = out[2];
  d[3] = out[3];
}


template <int KIND, int EPI>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(const GemmArgs pa, const GemmArgs pb,
                                                           int split, int nba, int nbb) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDSP];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BR * LDSP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  int bx, by;
  tile_of_block(bx, by);
  const bool second = bx >= split;
  const GemmArgs p = second ? pb : pa;
  int expert, row0, m_valid;
  if (!gemm_tile(p, bx, by, second, split, second ? nbb : nba, expert, row0, m_valid)) return;
  const int ntile = by;

  // ---- per-thread weight row (load stage): row r = tid/2, inputs 32*half.. of a K step
  const int br = tid >> 1, half = tid & 1;
  int n;
  bool upper = false;
  if (EPI == kEpiSwiglu) {
    upper = br >= 64;
    n = ntile * 64 + (br & 63);
  } else {
    n = ntile * BR + br;
  }
  // Every load of the K loop is unconditional, so the compiler can count the loads in flight
  // and wait for exactly the stage it needs: rows past N load row N - 1 (and store zeros),
  // rows past m_valid load the tile's first row (their products are never stored).
  const bool bvalid = n < p.N;
  const int nl = bvalid ? n : p.N - 1;
  const uint32_t *wrow = nullptr;
  const uint16_t *srow = nullptr, *brow = nullptr, *drow = nullptr;
  if (KIND == kBDense) {
    drow = p.bd + (int64_t)nl * p.bd_row_stride;
  } else {
    wrow = (upper ? p.w1 : p.w0) + (int64_t)expert * p.w_expert_stride + (int64_t)nl * p.w_row_stride;
    const int64_t so = (int64_t)expert * p.sb_expert_stride + (int64_t)nl * p.sb_row_stride;
    srow = (upper ? p.s1 : p.s0) + so;
    brow = (upper ? p.b1 : p.b0) + so;
  }

  // two register stages: the loads of step k + 2 are issued while step k computes, so each
  // step has a step's worth of time more for its memory round trip.  The weights of steps 0
  // and 1 need only the expert, so they are issued before the activation rows' index loads.
  u32x4 areg[2][4];
  BRegs breg[2];
  const int k1 = min(BK, p.K - BK);
  load_b<KIND>(breg[0], wrow, srow, brow, drow, 0, half, p.group);
  load_b<KIND>(breg[1], wrow, srow, brow, drow, k1, half, p.group);

  // ---- per-thread activation rows (load stage): 4 chunks of 16 B
  const uint16_t *arow[4];
  const int acol = (tid & 7) * 8;
  {
    // each level of row indices in four loads issued together (one round trip per level)
    int src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (tid >> 3) + 32 * i;
      src[i] = row0 + (r < m_valid ? r : 0);
    }
    if (p.a_rows) {
      uint32_t tt[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) tt[i] = p.a_rows[src[i]];
#pragma unroll
      for (int i = 0; i < 4; ++i) src[i] = (int)(tt[i] / (uint32_t)p.a_div);
    }
    if (p.a_rows2) {
      uint32_t tt[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) tt[i] = p.a_rows2[src[i]];
#pragma unroll
      for (int i = 0; i < 4; ++i) src[i] = (int)tt[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = p.A + (int64_t)src[i] * p.lda + acol;
  }

  // ---- MFMA ownership
  const int nrb = (m_valid + 15) >> 4;
  int cb0, cb1;
  if (EPI == kEpiSwiglu) {
    cb0 = wave;
    cb1 = wave + 4;
  } else {
    cb0 = 2 * wave;
    cb1 = 2 * wave + 1;
  }
  f32x4 acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    acc[i][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto load_stage = [&](int k0, int b) {
#pragma unroll
    for (int i = 0; i < 4; ++i) areg[b][i] = *(const u32x4 *)(arow[i] + k0);
    load_b<KIND>(breg[b], wrow, srow, brow, drow, k0, half, p.group);
  };
  auto step = [&](int k0, int b) {
    __syncthreads();
    // only the row blocks the MFMAs read (small tiles skip most of the tile's LDS writes)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if ((tid >> 3) + 32 * i < nrb * 16) *(u32x4 *)(As + ((tid >> 3) + 32 * i) * LDSP + acol) = areg[b][i];
    store_b<KIND>(Bs + br * LDSP + 32 * half, breg[b], bvalid);
    __syncthreads();
    // past the last step the stage reloads the last step (never stored)
    load_stage(min(k0 + 2 * BK, p.K - BK), b);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int koff = kk * 32 + (lane >> 4) * 8;
      const bf16x8 bf0 = __builtin_bit_cast(bf16x8, *(const u32x4 *)(Bs + (cb0 * 16 + (lane & 15)) * LDSP + koff));
      const bf16x8 bf1 = __builtin_bit_cast(bf16x8, *(const u32x4 *)(Bs + (cb1 * 16 + (lane & 15)) * LDSP + koff));
#pragma unroll
      for (int rb = 0; rb < 8; ++rb) {
        if (rb < nrb) {
          const bf16x8 af = __builtin_bit_cast(bf16x8, *(const u32x4 *)(As + (rb * 16 + (lane & 15)) * LDSP + koff));
          acc[rb][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf0, acc[rb][0], 0, 0, 0);
          acc[rb][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf1, acc[rb][1], 0, 0, 0);
        }
      }
    }
  };

#pragma unroll
  for (int i = 0; i < 4; ++i) areg[0][i] = *(const u32x4 *)(arow[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) areg[1][i] = *(const u32x4 *)(arow[i] + k1);
  int k0 = 0;
  for (; k0 + 2 * BK <= p.K; k0 += 2 * BK) {
    step(k0, 0);
    step(k0 + BK, 1);
  }
  if (k0 < p.K) step(k0, 0);  // an odd number of K steps
  __builtin_amdgcn_s_waitcnt(0x0f70);  // the trailing reloads land before the workgroup ends

  // ---- epilogue: lane holds column (lane & 15), rows 4*(lane >> 4) + i of each block
#pragma unroll
  for (int rb = 0; rb < 8; ++rb) {
    if (rb >= nrb) continue;
    // the block's four scattered destination rows, loaded together (one round trip)
    int dsts[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * 16 + (lane >> 4) * 4 + i;
      const int gr = row0 + (r < m_valid ? r : 0);
      dsts[i] = p.c_rows ? (int)p.c_rows[gr] : gr;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * 16 + (lane >> 4) * 4 + i;
      if (r >= m_valid) continue;
      const int dst = dsts[i];
      uint16_t *crow = p.C + (int64_t)dst * p.ldc;
      if (EPI == kEpiSwiglu) {
        const int col = ntile * 64 + wave * 16 + (lane & 15);
        if (col < p.N) {
          const float g = round_bf(acc[rb][0][i]);
          const float u = round_bf(acc[rb][1][i]);
          crow[col] = (uint16_t)swiglu_bf(g, u);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int col = ntile * BR + (c ? cb1 : cb0) * 16 + (lane & 15);
          if (col < p.N) {
            float v = acc[rb][c][i];
            if (EPI == kEpiBias) v = round_bf(v) + bf2f(p.bias[col]);
            crow[col] = (uint16_t)f2bf(v);
          }
        }
      }
    }
  }
}

template <int KIND>
hipError_t launch_kind(const GemmArgs &a, const GemmArgs *b, int epi, hipStream_t s) {
  auto shape = [&](const GemmArgs &g, int &mt, int &nb) {
    nb = epi == kEpiSwiglu ? (g.N + 63) / 64 : (g.N + BR - 1) / BR;
    mt = g.tile_expert ? g.max_tiles : (g.M + BM - 1) / BM;
    // all column tiles of one row tile land on the same XCD (blocks are dealt to the 8
    // XCDs round-robin by linear id) when the row-tile counts are multiples of 8
    mt = mt > 0 && nb > 0 ? (mt + 7) & ~7 : 0;
  };
  int mta, nba, mtb = 0, nbb = 0;
  shape(a, mta, nba);
  if (b) shape(*b, mtb, nbb);
  if (mta + mtb == 0) return hipSuccess;
  const GemmArgs &bb = b ? *b : a;
  dim3 grid(mta + mtb, std::max(nba, nbb)), block(256);
  if (epi == kEpiSwiglu)
    hipLaunchKernelGGL((grouped_gemm_kernel<KIND, kEpiSwiglu>), grid, block, 0, s, a, bb, mta, nba, nbb);
  else if (epi == kEpiBias)
    hipLaunchKernelGGL((grouped_gemm_kernel<KIND, kEpiBias>), grid, block, 0, s, a, bb, mta, nba, nbb);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<KIND, kEpiPlain>), grid, block, 0, s, a, bb, mta, nba, nbb);
  return hipGetLastError();
}


// 4 words of codes (32 inputs, 4-bit, LSB first) -> 4 chunks of 8 bf16, the words'
// conversions interleaved (each byte position converts 8 independent values) so that
// dependent instructions are several issues apart.  The nibble masks go through asm so that
// the compiler keeps them as one AND each and converts every byte with one
// v_cvt_f32_ubyte{0..3} (it would otherwise re-derive each nibble with a bit-field extract).
__device__ __forceinline__ void dequant32_q4(const u32x4 &q, float s, float b, u32x4 (&o)[4]) {
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo[w]) : "v"(q[w]));
#pragma unroll
  for (int w = 0; w < 4; ++w) asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi[w]) : "v"(q[w] >> 4));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float f0[4], f1[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      f0[w] = __builtin_fmaf(s, (float)((lo[w] >> (8 * i)) & 255u), b);
      f1[w] = __builtin_fmaf(s, (float)((hi[w] >> (8 * i)) & 255u), b);
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w][i] = pack_bf2_hw(f0[w], f1[w]);
  }
}

// ---------------------------------------------------------------- warp-specialised GEMM
//
// 4-bit affine weights, K a multiple of 64, groups of >= 32 inputs (an even number per
// row).  A workgroup of 12 waves owns one tile of up to 128 rows of one expert and 256
// weight rows (plain: 256 output columns; SwiGLU: 128 activated columns = 128 gate + 128
// up rows), stepping K by 64.  The waves specialise:
//   - producers (waves 0-7; wave w owns weight rows 32 w .. +32, two lanes per row) issue
//     the direct global->LDS loads of the activation tile, the codes and the scales /
//     biases two steps ahead, and turn step k+1's codes into a bf16 weight tile in LDS
//     (lane l: weight row 32 w + l / 2, inputs 32 (l % 2) .. +32 of the step);
//   - consumers (waves 8-11) run the MFMAs of step k: wave 8 + c owns weight rows
//     64 c .. +64 and every row block of the tile.
// One s_barrier per step separates the roles' uses of the rings (A, codes, scales: 3 slots;
// bf16 weights: 2 slots), so each SIMD runs two producers' dequantisation (two waves issue
// VALU work at twice the rate of one) next to a consumer's MFMAs.  Producers wait for their own loads with explicit vmcnt counts; no
// register loads happen inside the loop, so the compiler adds no waits of its own.
// LDS rows are 128 B (64 bf16) with 16-B chunk c of row r at position c ^ ((r >> 1) & 7),
// which spreads the 16 rows of an MFMA fragment over all 64 banks.
constexpr int WK = 64;                         // K step
constexpr int WNB = 256;                       // weight rows per workgroup
constexpr int WPW = 8;                         // producer waves (32 weight rows each)
constexpr int WA_SLOT = 128 * WK * 2;          // 16 KB: activation tile
constexpr int WC_SLOT = WNB * WK / 2;          // 8 KB: 4-bit codes
constexpr int WS_SLOT = 2 * WNB * 4;           // 2 KB: one dword of scales, one of biases
constexpr int WB_SLOT = WNB * WK * 2;          // 32 KB: bf16 weight tile
constexpr int WOFF_C = 3 * WA_SLOT, WOFF_S = WOFF_C + 3 * WC_SLOT, WOFF_B = WOFF_S + 3 * WS_SLOT;
constexpr int kWsLds = WOFF_B + 2 * WB_SLOT;   // 142 KB

__device__ __forceinline__ int wswz(int r, int c) { return c ^ ((r >> 1) & 7); }

// consumer: MFMAs of one K step over the wave's 4 column blocks and the tile's first 2 * NB
// 16-row blocks, in blocks of two row blocks (sub-step 0 then 1, so an accumulator is reused
// eight MFMAs later).  The step's B fragments are read first; each row-block pair's A
// fragments are read one pair ahead, so LDS latency hides behind the MFMAs.
template <int NB>
__device__ __forceinline__ void ws_mfma_step(const char *as, const char *bs, int cw, int lane,
                                             f32x4 (&acc)[8][4]) {
  const int c16 = lane & 15, kq = lane >> 4;
  bf16x8 bf[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const int n = cw * 64 + f * 16 + c16;
      bf[j][f] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(bs + n * 128 + 16 * wswz(n, 4 * j + kq)));
    }
  bf16x8 fa[2][2][2];  // [buffer][j][row block of the pair]
  auto read_blk = [&](int blk, int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r2 = 0; r2 < 2; ++r2) {
        const int r = (2 * blk + r2) * 16 + c16;
        fa[buf][j][r2] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(as + r * 128 + 16 * wswz(r, 4 * j + kq)));
      }
  };
  read_blk(0, 0);
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) {
    if (blk + 1 < NB) read_blk(blk + 1, (blk + 1) & 1);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int j = u >> 3, r2 = (u >> 2) & 1, f = u & 3;
      const int rb = 2 * blk + r2;
      acc[rb][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[blk & 1][j][r2], bf[j][f], acc[rb][f], 0, 0, 0);
    }
  }
}

template <int EPI>
__global__ __launch_bounds__(64 * (WPW + 4)) void ws_gemm_kernel(const GemmArgs pa, const GemmArgs pb, int split,
                                                      int nba, int nbb) {
  extern __shared__ __attribute__((aligned(16))) char ws_lds[];
  typedef __attribute__((address_space(3))) void lds_void;
  int bx, by;
  tile_of_block(bx, by);
  const bool second = bx >= split;
  const GemmArgs p = second ? pb : pa;
  int expert, row0, m_valid;
  if (!gemm_tile(p, bx, by, second, split, second ? nbb : nba, expert, row0, m_valid)) return;
  const int nblk = by;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nk = p.K / WK;
  const int lgg = __builtin_ctz((unsigned)p.group);  // group size: a power of two >= 32
  const bool producer = wave < WPW;

  if (producer) {
    // ---- this lane's weight row t and half hf (inputs 32 hf .. +32 of each step)
    const int t = wave * 32 + (lane >> 1), hf = lane & 1;
    // SwiGLU: consumer block t / 64 holds 32 gate rows (even producer wave) then the 32 up
    // rows of the same columns (odd producer wave)
    const bool upper = EPI == kEpiSwiglu && (wave & 1);
    auto row_of = [&](int tt) {
      const int n = EPI == kEpiSwiglu ? nblk * (WNB / 2) + (tt >> 6) * 32 + (tt & 31) : nblk * WNB + tt;
      return n < p.N ? n : p.N - 1;  // rows past N load a valid row; never stored
    };
    const uint32_t *wrow = (upper ? p.w1 : p.w0) + (int64_t)expert * p.w_expert_stride +
                           (int64_t)row_of(t) * p.w_row_stride + 4 * hf;
    // scale / bias loads: lane l < 32 fetches the scale dword of row 32 w + l, lane 32 + l
    // the bias dword of the same row
    const int64_t so = (int64_t)expert * p.sb_expert_stride + (int64_t)row_of(wave * 32 + (lane & 31)) * p.sb_row_stride;
    const uint16_t *sbrow = (lane < 32 ? (upper ? p.s1 : p.s0) : (upper ? p.b1 : p.b0)) + so;
    // ---- A rows: load v of producer wave w fills rows (v * WPW + w) * 8 + lane / 8, position
    // lane % 8 (holding K chunk wswz(row, lane % 8))
    constexpr int AV = 16 / WPW;
    const uint16_t *asrc[AV];
    {
      int src[AV];
#pragma unroll
      for (int v = 0; v < AV; ++v) {
        const int r = (v * WPW + wave) * 8 + (lane >> 3);
        src[v] = row0 + (r < m_valid ? r : 0);
      }
      if (p.a_rows) {
        uint32_t tt[AV];
#pragma unroll
        for (int v = 0; v < AV; ++v) tt[v] = p.a_rows[src[v]];
#pragma unroll
        for (int v = 0; v < AV; ++v) src[v] = (int)(tt[v] / (uint32_t)p.a_div);
      }
      if (p.a_rows2) {
        uint32_t tt[AV];
#pragma unroll
        for (int v = 0; v < AV; ++v) tt[v] = p.a_rows2[src[v]];
#pragma unroll
        for (int v = 0; v < AV; ++v) src[v] = (int)tt[v];
      }
#pragma unroll
      for (int v = 0; v < AV; ++v) {
        const int r = (v * WPW + wave) * 8 + (lane >> 3);
        asrc[v] = p.A + (int64_t)src[v] * p.lda + 8 * wswz(r, lane & 7);
      }
    }
    auto issue_a = [&](int k, int nav) {  // nav (a constant at each call) loads
      const int kc = k < nk ? k : nk - 1;
      char *base = ws_lds + (k % 3) * WA_SLOT;
#pragma unroll
      for (int v = 0; v < AV; ++v)
        if (v < nav) __builtin_amdgcn_global_load_lds((const void *)(asrc[v] + kc * WK),
                                         (lds_void *)(base + (v * WPW + wave) * 1024), 16, 0, 0);
    };
    auto issue_c = [&](int k) {  // 2 loads: codes (16 B per lane), the scale / bias dwords
      const int kc = k < nk ? k : nk - 1;
      const int k0 = kc * WK;
      char *cb = ws_lds + WOFF_C + (k % 3) * WC_SLOT;
      __builtin_amdgcn_global_load_lds((const void *)(wrow + k0 / 8), (lds_void *)(cb + wave * 1024), 16, 0, 0);
      const int gd = (k0 >> lgg) & ~1;  // dword holding the step's first group
      char *sb = ws_lds + WOFF_S + (k % 3) * WS_SLOT;
      __builtin_amdgcn_global_load_lds((const void *)(sbrow + gd), (lds_void *)(sb + wave * 256), 4, 0, 0);
    };
    auto dequant = [&](int k) {  // codes of step k -> bf16 slot k % 2
      const char *cb = ws_lds + WOFF_C + (k % 3) * WC_SLOT;
      const char *sb = ws_lds + WOFF_S + (k % 3) * WS_SLOT;
      const uint32_t sw = *(const uint32_t *)(sb + wave * 256 + (lane >> 1) * 4);
      const uint32_t bw = *(const uint32_t *)(sb + wave * 256 + 128 + (lane >> 1) * 4);
      const u32x4 q = *(const u32x4 *)(cb + wave * 1024 + lane * 16);
      const int k0 = k * WK;
      // group of inputs k0 + 32 hf .. +32, relative to the dword's first group
      const int gi = ((k0 + 32 * hf) >> lgg) - ((k0 >> lgg) & ~1);
      const float sc = gi ? bf_hi(sw) : bf_lo(sw);
      const float bi = gi ? bf_hi(bw) : bf_lo(bw);
      char *bs = ws_lds + WOFF_B + (k & 1) * WB_SLOT;
      u32x4 o[4];
      dequant32_q4(q, sc, bi, o);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int c = hf * 4 + w;  // 16-B chunk of the row: inputs 8c .. 8c+7
        *(u32x4 *)(bs + t * 128 + 16 * wswz(t, c)) = o[w];
      }
    };
    // NA activation loads per step: a tile of at most 64 rows loads only rows 0-63 (load 0
    // of every producer wave), the rows its consumers read
    auto run = [&](auto na_tag) {
      constexpr int NA = decltype(na_tag)::value, NC = 2;
      // prologue: codes 0, then [A 0, codes 1], [A 1, codes 2]
      issue_c(0);
      issue_a(0, NA);
      issue_c(1);
      issue_a(1, NA);
      issue_c(2);
      wait_vmcnt_le(2 * (NA + NC));  // codes 0
      dequant(0);
      wait_vmcnt_le(NA + 2 * NC);    // A 0
      ring_barrier();
      for (int k = 0; k < nk; ++k) {
        // step k: the consumers compute step k
        wait_vmcnt_le(NA + NC);       // codes k + 1
        if (k + 1 < nk) dequant(k + 1);
        issue_a(k + 2, NA);
        issue_c(k + 3);
        wait_vmcnt_le(NA + 2 * NC);   // A k + 1
        ring_barrier();
      }
    };
    if (m_valid <= 64) run(std::integral_constant<int, 1>());
    else run(std::integral_constant<int, AV>());
    __builtin_amdgcn_s_waitcnt(0x0f70);  // drain the clamped trailing loads
    return;
  }

  // ---- consumers
  const int cw = wave - WPW;
  f32x4 acc[8][4];
#pragma unroll
  for (int rb = 0; rb < 8; ++rb)
#pragma unroll
    for (int f = 0; f < 4; ++f) acc[rb][f] = f32x4{0.f, 0.f, 0.f, 0.f};
  ring_barrier();  // step 0's A and weights are ready
  // row-block pairs the tile needs: 64, 96 or 128 rows (about half of the experts of a
  // uniform 2048-token prefill hold 65-96 rows, which then skip a quarter of the MFMAs)
  const int nbu = m_valid <= 64 ? 2 : m_valid <= 96 ? 3 : 4;
  auto consume = [&](auto nb_tag) {
    constexpr int NB = decltype(nb_tag)::value;
    for (int k = 0; k < nk; ++k) {
      const char *as = ws_lds + (k % 3) * WA_SLOT;
      const char *bs = ws_lds + WOFF_B + (k & 1) * WB_SLOT;
      ws_mfma_step<NB>(as, bs, cw, lane, acc);
      ring_barrier();
    }
  };
  if (nbu == 2) consume(std::integral_constant<int, 2>());
  else if (nbu == 3) consume(std::integral_constant<int, 3>());
  else consume(std::integral_constant<int, 4>());

  // ---- epilogue: lane holds column (lane & 15) of each block, rows 4 (lane >> 4) + i
  const int c16 = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int rb = 0; rb < 8; ++rb) {
    if (rb >= 2 * nbu) break;
    // the block's four scattered destination rows, loaded together (one round trip)
    int dsts[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * 16 + kq * 4 + i;
      const int gr = row0 + (r < m_valid ? r : 0);
      dsts[i] = p.c_rows ? (int)p.c_rows[gr] : gr;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * 16 + kq * 4 + i;
      if (r >= m_valid) continue;
      const int dst = dsts[i];
      uint16_t *crow = p.C + (int64_t)dst * p.ldc;
      if (EPI == kEpiSwiglu) {
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const int col = nblk * (WNB / 2) + cw * 32 + f * 16 + c16;
          if (col < p.N) {
            const float g = round_bf(acc[rb][f][i]);
            const float u = round_bf(acc[rb][f + 2][i]);
            crow[col] = (uint16_t)swiglu_bf(g, u);
          }
        }
      } else {
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const int col = nblk * WNB + cw * 64 + f * 16 + c16;
          if (col < p.N) {
            float v = acc[rb][f][i];
            if (EPI == kEpiBias) v = round_bf(v) + bf2f(p.bias[col]);
            crow[col] = (uint16_t)f2bf(v);
          }
        }
      }
    }
  }
}


hipError_t launch_ws(const GemmArgs &a, const GemmArgs *b, int epi, hipStream_t s) {
  auto shape = [&](const GemmArgs &g, int &mt, int &nb) {
    nb = epi == kEpiSwiglu ? (g.N + WNB / 2 - 1) / (WNB / 2) : (g.N + WNB - 1) / WNB;
    mt = g.tile_expert ? g.max_tiles : (g.M + BM - 1) / BM;
    mt = mt > 0 && nb > 0 ? (mt + 7) & ~7 : 0;  // one XCD per row tile (see launch_kind)
  };
  int mta, nba, mtb = 0, nbb = 0;
  shape(a, mta, nba);
  if (b) shape(*b, mtb, nbb);
  if (mta + mtb == 0) return hipSuccess;
  const GemmArgs &bb = b ? *b : a;
  dim3 grid(mta + mtb, std::max(nba, nbb)), block(64 * (WPW + 4));
  static bool raised[3] = {false, false, false};  // > 64 KB of LDS is an opt-in per kernel
  auto launch = [&](auto kernel, int which) {
    if (!raised[which]) {
      const hipError_t e = hipFuncSetAttribute((const void *)kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kWsLds);
      if (e != hipSuccess) return e;
      raised[which] = true;
    }
    hipLaunchKernelGGL(kernel, grid, block, kWsLds, s, a, bb, mta, nba, nbb);
    return hipGetLastError();
  };
  if (epi == kEpiSwiglu) return launch(ws_gemm_kernel<kEpiSwiglu>, 0);
  if (epi == kEpiBias) return launch(ws_gemm_kernel<kEpiBias>, 1);
  return launch(ws_gemm_kernel<kEpiPlain>, 2);
}

// Dense bf16 weights over one implicit group of rows (the router projection at prefill
// sizes, N = experts is small): a 32-row x 64-column output tile per 4-wave workgroup, so
// that even N = 256 gives M / 32 * 4 workgroups.  K advances 128 at a time through 4 LDS
// stages (96 KB) filled three steps ahead by direct global->LDS loads in which 16
// consecutive lanes read one row's 256 bytes (a fragment-shaped register load, 16 rows per
// instruction, keeps the texture addresser busy one lane per cycle).  LDS rows are 256 B
// with 16-B chunk c of row r at position c ^ (r & 15), so the 16 rows of a fragment read hit
// 16 different 16-B bank groups; wave w owns columns 16 w .. +16 of the tile and both
// 16-row blocks.  Workgroups of one 32-row block share an XCD.
constexpr int DT_M = 32, DT_N = 64, DT_K = 128, DT_STAGES = 4, DT_J = DT_K / 32;
constexpr int DT_ROW = DT_K * 2;                                          // 256 B
constexpr int DT_ASLOT = DT_M * DT_ROW, DT_BSLOT = DT_N * DT_ROW;        // 8 KB, 16 KB
constexpr int DT_SLOT = DT_ASLOT + DT_BSLOT;
constexpr int kDenseLds = DT_STAGES * DT_SLOT;                            // 96 KB
constexpr int DT_LOADS = (DT_M + DT_N) * DT_ROW / 1024 / 4;               // per wave per stage: 6

__device__ __forceinline__ int dswz(int r, int c) { return c ^ (r & 15); }

template <int EPI>
__global__ __launch_bounds__(256) void dense_gemm_kernel(const GemmArgs p, int nrb, int ncb) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  typedef __attribute__((address_space(3))) void lds_void;
  const int blk = blockIdx.x;
  const int rb = (blk & 7) + 8 * (blk / (8 * ncb));
  const int cb = (blk >> 3) % ncb;
  if (rb >= nrb) return;  // grid padding to whole rounds of 8 row blocks
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nk = p.K / DT_K;
  // load i of this wave covers tile row 4 (6 wave + i) + lane / 16 of the stage (rows 0-31:
  // A, rows 32-95: B), LDS position lane % 16 holding chunk dswz(row, lane % 16)
  const int lr = lane >> 4, lp = lane & 15;
  const uint16_t *src[DT_LOADS];
#pragma unroll
  for (int i = 0; i < DT_LOADS; ++i) {
    const int tr = 4 * (DT_LOADS * wave + i) + lr;
    if (tr < DT_M) {
      const int gr = rb * DT_M + tr;
      src[i] = p.A + (int64_t)(gr < p.M ? gr : p.M - 1) * p.lda + 8 * dswz(tr, lp);
    } else {
      const int n = tr - DT_M, g = cb * DT_N + n;
      src[i] = p.bd + (int64_t)(g < p.N ? g : p.N - 1) * p.bd_row_stride + 8 * dswz(n, lp);
    }
  }
  auto issue = [&](int k) {  // stage k (clamped to the last step) into its slot
    const int kc = (k < nk ? k : nk - 1) * DT_K;
    char *slot = lds + (k % DT_STAGES) * DT_SLOT;
#pragma unroll
    for (int i = 0; i < DT_LOADS; ++i)
      __builtin_amdgcn_global_load_lds((const void *)(src[i] + kc),
                                       (lds_void *)(slot + (DT_LOADS * wave + i) * 1024), 16, 0, 0);
  };
  const int c16 = lane & 15, kq = lane >> 4;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < DT_STAGES - 1; ++k) issue(k);
  for (int k = 0; k < nk; ++k) {
    wait_vmcnt_le(DT_LOADS * (DT_STAGES - 2));  // this wave's loads of stage k
    ring_barrier();  // every wave's loads of stage k are in LDS; stage k - 1 is consumed
    issue(k + DT_STAGES - 1);
    const char *as = lds + (k % DT_STAGES) * DT_SLOT, *bs = as + DT_ASLOT;
    bf16x8 fa[DT_J][2], fb[DT_J];
    const int n = wave * 16 + c16, r0 = c16, r1 = 16 + c16;
#pragma unroll
    for (int j = 0; j < DT_J; ++j) {
      fb[j] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(bs + n * DT_ROW + 16 * dswz(n, 4 * j + kq)));
      fa[j][0] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(as + r0 * DT_ROW + 16 * dswz(r0, 4 * j + kq)));
      fa[j][1] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(as + r1 * DT_ROW + 16 * dswz(r1, 4 * j + kq)));
    }
#pragma unroll
    for (int j = 0; j < DT_J; ++j) {
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[j][0], fb[j], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[j][1], fb[j], acc1, 0, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // drain the clamped trailing loads
  // lane holds column c16 of rows 4 kq + i of each 16-row block
  const int n = cb * DT_N + wave * 16 + c16;
  if (n >= p.N) return;
  const float bias = EPI == kEpiBias ? bf2f(p.bias[n]) : 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * DT_M + h * 16 + kq * 4 + i;
      if (r >= p.M) continue;
      float v = h ? acc1[i] : acc0[i];
      if (EPI == kEpiBias) v = round_bf(v) + bias;
      p.C[(int64_t)r * p.ldc + n] = (uint16_t)f2bf(v);
    }
  }
}

hipError_t launch_dense(const GemmArgs &a, int epi, hipStream_t s) {
  const int nrb = (a.M + DT_M - 1) / DT_M, ncb = (a.N + DT_N - 1) / DT_N;
  const int grid = ((nrb + 7) & ~7) * ncb;
  static bool raised[2] = {false, false};  // > 64 KB of LDS is an opt-in per kernel
  auto launch = [&](auto kernel, int which) {
    if (!raised[which]) {
      const hipError_t e = hipFuncSetAttribute((const void *)kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kDenseLds);
      if (e != hipSuccess) return e;
      raised[which] = true;
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), kDenseLds, s, a, nrb, ncb);
    return hipGetLastError();
  };
  if (epi == kEpiBias) return launch(dense_gemm_kernel<kEpiBias>, 0);
  return launch(dense_gemm_kernel<kEpiPlain>, 1);
}

// ---------------------------------------------------------------- affine rows, exact codes
//
// Affine weights over one implicit group of rows with the codes exact on the MFMA (the router
// projection of an affine router, quantized_linear, forward.rs:53-58, at prefill sizes).  A
// 32-input MFMA step never crosses an affine group (g >= 32), so each group's sum is
//   sum_k x (s q + b) = s * sum_k x (MAG + q) + (b - MAG s) * sum_k x,
// with MAG + q made exact in bf16 by OR-ing the 4-bit code into the mantissa of 128 (8-bit
// codes convert exactly, MAG = 0) and sum_k x from an MFMA against ones; the affine terms are
// applied to the group's fp32 partial sums once per group.  No weight is rounded to bf16 (the
// grouped GEMMs round dequantised weights before their MFMAs), so the logits stay within about
// one bf16 ulp of an fp32 dequantise-and-dot, as the decode kernels' router does.
// Tile: 32 rows x 64 weight rows per 4-wave workgroup, K steps of 128 staged in LDS with the
// next step's loads in registers during the current step's MFMAs; wave w owns weight rows
// 16 w .. +16 of the tile and both 16-row blocks.
constexpr int AQ_M = 32, AQ_N = 64, AQ_K = 128, AQ_J = AQ_K / 32;

template <int BITS>
__device__ __forceinline__ int aq_swz(int n) {  // 16-B piece XOR of weight row n (64 / 128-B rows)
  return BITS == 4 ? ((n >> 2) & 3) : ((n >> 1) & 7);
}

template <int BITS, int EPI>
__global__ __launch_bounds__(256) void affine_rows_gemm_kernel(const GemmArgs p, int nrb, int ncb) {
  constexpr int BROW = AQ_K * BITS / 8;         // code bytes per weight row per step: 64 / 128
  constexpr int BPC = BROW / 16;                // 16-B pieces per weight row
  constexpr int BLD = AQ_N * BPC / 256;         // code pieces per thread per step: 1 / 2
  constexpr float MAG = BITS == 4 ? 128.0f : 0.0f;
  __shared__ __attribute__((aligned(16))) char As[AQ_M * AQ_K * 2];  // 256-B rows, chunk c at c ^ (r & 15)
  __shared__ __attribute__((aligned(16))) char Bs[AQ_N * BROW];
  __shared__ float Ss[AQ_N][AQ_J], Cs[AQ_N][AQ_J];  // s and b - MAG s of each 32-input step's group
  const int blk = blockIdx.x;
  const int rb = (blk & 7) + 8 * (blk / (8 * ncb));
  const int cb = (blk >> 3) % ncb;
  if (rb >= nrb) return;  // grid padding to whole rounds of 8 row blocks
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nk = p.K / AQ_K;
  // this thread's loads of a step: two 16-B pieces of activations, BLD of codes, one (s, b)
  const uint16_t *asrc[2];
  int adst[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + 256 * i, r = q >> 4, pc = q & 15;
    const int gr = rb * AQ_M + r;
    asrc[i] = p.A + (int64_t)(gr < p.M ? gr : p.M - 1) * p.lda + 8 * pc;
    adst[i] = r * 256 + 16 * (pc ^ (r & 15));
  }
  const uint32_t *bsrc[BLD];
  int bdst[BLD];
#pragma unroll
  for (int i = 0; i < BLD; ++i) {
    const int q = tid + 256 * i, n = q / BPC, pc = q % BPC;
    const int gn = cb * AQ_N + n;
    bsrc[i] = p.w0 + (int64_t)(gn < p.N ? gn : p.N - 1) * p.w_row_stride + 4 * pc;
    bdst[i] = n * BROW + 16 * (pc ^ aq_swz<BITS>(n));
  }
  const int sn = tid >> 2, sj = tid & 3;  // (weight row, 32-input step) of the (s, b) load
  const int64_t sbo = (int64_t)(cb * AQ_N + sn < p.N ? cb * AQ_N + sn : p.N - 1) * p.sb_row_stride;
  const uint16_t *srow = p.s0 + sbo, *brow = p.b0 + sbo;
  u32x4 ra[2], rbq[BLD];
  uint16_t rs, rbias;
  auto load = [&](int k) {
    const int k0 = k * AQ_K;
#pragma unroll
    for (int i = 0; i < 2; ++i) ra[i] = *(const u32x4 *)(asrc[i] + k0);
#pragma unroll
    for (int i = 0; i < BLD; ++i) rbq[i] = *(const u32x4 *)(bsrc[i] + k0 * BITS / 32);
    const int gi = (k0 + 32 * sj) / p.group;
    rs = srow[gi];
    rbias = brow[gi];
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) *(u32x4 *)(As + adst[i]) = ra[i];
#pragma unroll
    for (int i = 0; i < BLD; ++i) *(u32x4 *)(Bs + bdst[i]) = rbq[i];
    const float sv = bf2f(rs);
    Ss[sn][sj] = sv;
    Cs[sn][sj] = __builtin_fmaf(-MAG, sv, bf2f(rbias));
  };
  const int c16 = lane & 15, kq = lane >> 4;
  const int n = wave * 16 + c16;  // this lane's weight row in the tile
  const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[2] = {zero, zero}, part[2] = {zero, zero}, xs[2] = {zero, zero};
  load(0);
  store();
  __syncthreads();
  for (int k = 0; k < nk; ++k) {
    if (k + 1 < nk) load(k + 1);
#pragma unroll
    for (int j = 0; j < AQ_J; ++j) {
      u32x4 b;
      if constexpr (BITS == 4) {
        const uint32_t wd = *(const uint32_t *)(Bs + n * BROW + 16 * (j ^ aq_swz<4>(n)) + 4 * kq);
        b[0] = (wd & 0x000f000fu) | 0x43004300u;  // inputs (8 kq + i, 8 kq + i + 4) as 128 + q
        b[1] = ((wd >> 4) & 0x000f000fu) | 0x43004300u;
        b[2] = ((wd >> 8) & 0x000f000fu) | 0x43004300u;
        b[3] = ((wd >> 12) & 0x000f000fu) | 0x43004300u;
      } else {
        const uint2 raw = *(const uint2 *)(Bs + n * BROW + 16 * ((2 * j + (kq >> 1)) ^ aq_swz<8>(n)) + 8 * (kq & 1));
        const uint32_t w2[2] = {raw.x, raw.y};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t v = w2[h];
          b[2 * h] = pack_bf2_hw((float)(v & 255u), (float)((v >> 8) & 255u));
          b[2 * h + 1] = pack_bf2_hw((float)((v >> 16) & 255u), (float)(v >> 24));
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = h * 16 + c16;
        u32x4 a = *(const u32x4 *)(As + r * 256 + 16 * ((4 * j + kq) ^ (r & 15)));
        if constexpr (BITS == 4) {  // (x0, x4), (x1, x5), (x2, x6), (x3, x7): the codes' pairing
          const u32x4 d = a;
          a[0] = (d[0] & 0xffffu) | (d[2] << 16);
          a[1] = (d[0] >> 16) | (d[2] & 0xffff0000u);
          a[2] = (d[1] & 0xffffu) | (d[3] << 16);
          a[3] = (d[1] >> 16) | (d[3] & 0xffff0000u);
        }
        part[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                          part[h], 0, 0, 0);
        xs[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, ones),
                                                        xs[h], 0, 0, 0);
      }
      if ((k * AQ_K + 32 * (j + 1)) % p.group == 0) {  // the group ends with this step
        const float sv = Ss[n][j], cv = Cs[n][j];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[h][i] = __builtin_fmaf(cv, xs[h][i], __builtin_fmaf(sv, part[h][i], acc[h][i]));
          part[h] = zero;
          xs[h] = zero;
        }
      }
    }
    __syncthreads();
    if (k + 1 < nk) {
      store();
      __syncthreads();
    }
  }
  // lane holds column c16 of rows 4 kq + i of each 16-row block
  const int col = cb * AQ_N + n;
  if (col >= p.N) return;
  const float bias = EPI == kEpiBias ? bf2f(p.bias[col]) : 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * AQ_M + h * 16 + kq * 4 + i;
      if (r >= p.M) continue;
      float v = acc[h][i];
      if (EPI == kEpiBias) v = round_bf(v) + bias;
      p.C[(int64_t)r * p.ldc + col] = (uint16_t)f2bf(v);
    }
  }
}

bool use_dense(const GemmArgs &a, int epi) {
  // one implicit group, bf16 weights, 16-B aligned 64-input steps, no row indirection
  return a.bkind == kBDense && !a.tile_expert && !a.a_rows && !a.c_rows && epi != kEpiSwiglu &&
         a.K % DT_K == 0 && a.lda % 8 == 0 && a.bd_row_stride % 8 == 0 && a.M > 0 && a.N > 0 &&
         ((uintptr_t)a.A & 15) == 0 && ((uintptr_t)a.bd & 15) == 0;
}

bool use_ws(const GemmArgs &a) {
  // 4-bit weights with K steps of 64 and an even number of groups of >= 32 inputs per row
  // (one dword of scales per step stays 4-byte aligned); K >= 1024: with fewer K steps its
  // two-step prefetch ramp outweighs the gain
  return a.bkind == kBQ4 && a.K % WK == 0 && a.K >= 1024 && a.group >= 32 &&
         (a.group & (a.group - 1)) == 0 && (a.K / a.group) % 2 == 0;
}

}  // namespace

bool affine_rows_supported(const GemmArgs &a, int epilogue) {
  return (a.bkind == kBQ4 || a.bkind == kBQ8) && !a.tile_expert && !a.a_rows && !a.a_rows2 && !a.c_rows &&
         epilogue != kEpiSwiglu && a.K % AQ_K == 0 && a.group >= 32 && a.lda % 8 == 0 &&
         a.w_row_stride % 4 == 0 && a.M > 0 && a.N > 0 && ((uintptr_t)a.A & 15) == 0 &&
         ((uintptr_t)a.w0 & 15) == 0;
}

hipError_t launch_affine_rows(const GemmArgs &a, int epilogue, hipStream_t s) {
  const int nrb = (a.M + AQ_M - 1) / AQ_M, ncb = (a.N + AQ_N - 1) / AQ_N;
  const int grid = ((nrb + 7) & ~7) * ncb;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, s, a, nrb, ncb);
    return hipGetLastError();
  };
  if (a.bkind == kBQ8)
    return epilogue == kEpiBias ? go(affine_rows_gemm_kernel<8, kEpiBias>) : go(affine_rows_gemm_kernel<8, kEpiPlain>);
  return epilogue == kEpiBias ? go(affine_rows_gemm_kernel<4, kEpiBias>) : go(affine_rows_gemm_kernel<4, kEpiPlain>);
}

hipError_t launch_grouped_gemm(const GemmArgs &a, int epilogue, hipStream_t s) {
  return launch_grouped_gemm2(a, nullptr, epilogue, s);
}

bool gemm_fusable(const GemmArgs &a, const GemmArgs &b) {
  // one kernel instantiation serves both problems: the same kernel choice, and for the
  // exact-code kernel the same group size
  const bool xq = xq_supported(a);
  return a.bkind == b.bkind && xq == xq_supported(b) && (!xq || a.group == b.group) && use_ws(a) == use_ws(b);
}



hipError_t launch_grouped_gemm2(const GemmArgs &a, const GemmArgs *b, int epilogue, hipStream_t s) {
  if (b && !gemm_fusable(a, *b)) {
    const hipError_t e = launch_grouped_gemm2(a, nullptr, epilogue, s);
    return e == hipSuccess ? launch_grouped_gemm2(*b, nullptr, epilogue, s) : e;
  }
  if (!b && use_dense(a, epilogue)) return launch_dense(a, epilogue, s);
  if (xq_supported(a)) return launch_xq(a, b, epilogue, s);
  if (use_ws(a)) return launch_ws(a, b, epilogue, s);
  switch (a.bkind) {
    case kBQ4: return launch_kind<kBQ4>(a, b, epilogue, s);
    case kBQ8: return launch_kind<kBQ8>(a, b, epilogue, s);
    default: return launch_kind<kBDense>(a, b, epilogue, s);
  }
}

}  // namespace astro
