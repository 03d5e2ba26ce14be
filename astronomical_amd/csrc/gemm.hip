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
#include "kernels.h"

namespace astro {

namespace {

constexpr int BM = kGemmBM;  // rows per tile
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

struct BRegs {
  u32x4 q[4];
  float s, b;
};

template <int KIND>
__device__ __forceinline__ void load_b(BRegs &r, const uint32_t *wrow, const uint16_t *srow,
                                       const uint16_t *brow, const uint16_t *drow, int k0,
                                       int half, int group, bool valid) {
  if (!valid) return;
  if (KIND == kBQ4) {
    r.q[0] = *(const u32x4 *)(wrow + (k0 >> 3) + half * 4);
    const int g = (k0 + 32 * half) / group;
    r.s = bf2f(srow[g]);
    r.b = bf2f(brow[g]);
  } else if (KIND == kBQ8) {
    const u32x4 *p = (const u32x4 *)(wrow + (k0 >> 2) + half * 8);
    r.q[0] = p[0];
    r.q[1] = p[1];
    const int g = (k0 + 32 * half) / group;
    r.s = bf2f(srow[g]);
    r.b = bf2f(brow[g]);
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
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
      const uint32_t w = r.q[0][wi];
      uint32_t p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float q0 = (float)((w >> (8 * j)) & 15u);
        const float q1 = (float)((w >> (8 * j + 4)) & 15u);
        p[j] = pack_bf2_hw(__builtin_fmaf(r.s, q0, r.b), __builtin_fmaf(r.s, q1, r.b));
      }
      out[wi] = u32x4{p[0], p[1], p[2], p[3]};
    }
  } else if (KIND == kBQ8) {
#pragma unroll
    for (int wi = 0; wi < 8; ++wi) {
      const uint32_t w = r.q[wi >> 2][wi & 3];
      const float q0 = (float)(w & 255u), q1 = (float)((w >> 8) & 255u);
      const float q2 = (float)((w >> 16) & 255u), q3 = (float)(w >> 24);
      const uint32_t p0 = pack_bf2_hw(__builtin_fmaf(r.s, q0, r.b), __builtin_fmaf(r.s, q1, r.b));
      const uint32_t p1 = pack_bf2_hw(__builtin_fmaf(r.s, q2, r.b), __builtin_fmaf(r.s, q3, r.b));
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

template <int KIND, int EPI, bool GROUPED>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(const GemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDSP];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BR * LDSP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  int expert = 0, row0, m_valid;
  if (GROUPED) {
    const int tile = blockIdx.x;
    if (tile >= (int)*p.tile_count) return;
    expert = (int)p.tile_expert[tile];
    row0 = (int)p.tile_row0[tile];
    m_valid = min(BM, (int)p.expert_offsets[expert + 1] - row0);
  } else {
    row0 = blockIdx.x * BM;
    m_valid = min(BM, p.M - row0);
  }
  if (m_valid <= 0) return;
  const int ntile = blockIdx.y;

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
  const bool bvalid = n < p.N;
  const uint32_t *wrow = nullptr;
  const uint16_t *srow = nullptr, *brow = nullptr, *drow = nullptr;
  if (bvalid) {
    if (KIND == kBDense) {
      drow = p.bd + (int64_t)n * p.bd_row_stride;
    } else {
      wrow = (upper ? p.w1 : p.w0) + (int64_t)expert * p.w_expert_stride + (int64_t)n * p.w_row_stride;
      const int64_t so = (int64_t)expert * p.sb_expert_stride + (int64_t)n * p.sb_row_stride;
      srow = (upper ? p.s1 : p.s0) + so;
      brow = (upper ? p.b1 : p.b0) + so;
    }
  }

  // ---- per-thread activation rows (load stage): 4 chunks of 16 B
  const uint16_t *arow[4];
  const int acol = (tid & 7) * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 3) + 32 * i;
    arow[i] = nullptr;
    if (r < m_valid) {
      const int gr = row0 + r;
      int src = p.a_rows ? (int)(p.a_rows[gr] / (uint32_t)p.a_div) : gr;
      if (p.a_rows2) src = (int)p.a_rows2[src];
      arow[i] = p.A + (int64_t)src * p.lda + acol;
    }
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

  u32x4 areg[4];
  BRegs breg;
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      areg[i] = arow[i] ? *(const u32x4 *)(arow[i] + k0) : u32x4{0, 0, 0, 0};
    load_b<KIND>(breg, wrow, srow, brow, drow, k0, half, p.group, bvalid);
  };

  load_stage(0);
  for (int k0 = 0; k0 < p.K; k0 += BK) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *(u32x4 *)(As + ((tid >> 3) + 32 * i) * LDSP + acol) = areg[i];
    store_b<KIND>(Bs + br * LDSP + 32 * half, breg, bvalid);
    __syncthreads();
    if (k0 + BK < p.K) load_stage(k0 + BK);
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
  }

  // ---- epilogue: lane holds column (lane & 15), rows 4*(lane >> 4) + i of each block
#pragma unroll
  for (int rb = 0; rb < 8; ++rb) {
    if (rb >= nrb) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rb * 16 + (lane >> 4) * 4 + i;
      if (r >= m_valid) continue;
      const int gr = row0 + r;
      const int dst = p.c_rows ? (int)p.c_rows[gr] : gr;
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

template <int KIND, bool GROUPED>
hipError_t launch_kind(const GemmArgs &a, int epi, hipStream_t s) {
  const int ntiles = epi == kEpiSwiglu ? (a.N + 63) / 64 : (a.N + BR - 1) / BR;
  int mt = GROUPED ? a.max_tiles : (a.M + BM - 1) / BM;
  if (mt <= 0 || ntiles <= 0) return hipSuccess;
  // all column tiles of one row tile land on the same XCD (blocks are dealt to the 8
  // XCDs round-robin by linear id) when the row-tile count is a multiple of 8
  mt = (mt + 7) & ~7;
  dim3 grid(mt, ntiles), block(256);
  if (epi == kEpiSwiglu)
    hipLaunchKernelGGL((grouped_gemm_kernel<KIND, kEpiSwiglu, GROUPED>), grid, block, 0, s, a);
  else if (epi == kEpiBias)
    hipLaunchKernelGGL((grouped_gemm_kernel<KIND, kEpiBias, GROUPED>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<KIND, kEpiPlain, GROUPED>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <int KIND>
hipError_t launch_kind(const GemmArgs &a, int epi, hipStream_t s) {
  return a.tile_expert ? launch_kind<KIND, true>(a, epi, s) : launch_kind<KIND, false>(a, epi, s);
}

}  // namespace

hipError_t launch_grouped_gemm(const GemmArgs &a, int epilogue, hipStream_t s) {
  switch (a.bkind) {
    case kBQ4: return launch_kind<kBQ4>(a, epilogue, s);
    case kBQ8: return launch_kind<kBQ8>(a, epilogue, s);
    default: return launch_kind<kBDense>(a, epilogue, s);
  }
}

}  // namespace astro
