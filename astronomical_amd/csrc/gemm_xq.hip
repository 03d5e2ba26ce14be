// The exact-code grouped GEMM for 4-bit affine weights (and the activation rows' group sums
// it needs).  Built in its own object with MFMA results in VGPRs
// (-mllvm=-amdgpu-mfma-vgpr-form): the per-group affine terms are VALU work on the MFMA
// accumulators, which AGPRs would make cross the register files.
//
// No weight is dequantised.  A 32-input MFMA step never crosses an affine group, so a group's
// contribution to an output is
//   sum_k x (s q + b) = s * sum_k x (128 + q) + (b - 128 s) * sum_k x,
// the MFMA runs on the exact codes (128 + q is bf16 0x4300 | q: one AND-OR makes two of them)
// into a per-group fp32 partial P, and at the group's end acc += s P + (b - 128 s) X, with X the
// group's sum of the activation row (GemmArgs::xsum, from group_sums_kernel).  The cheap unpack
// pairs the codes of inputs (i, i + 4) of each 8-input word, so the activations take the same
// pairing: permuted in the A fragment, or already permuted in memory (GemmArgs::a_paired, the
// copy group_sums_kernel writes of x).
//
// A workgroup of 8 waves (one per CU) owns a tile of up to 64 rows of one expert and 512 weight
// rows (plain: 512 output columns; SwiGLU: 256 activated columns = 256 gate + 256 up rows), K
// stepped by 128.  Wave w owns weight rows 64 w .. +64 (SwiGLU: the gate rows, then the up
// rows, of 32 columns) and every row block of the tile, and unpacks its own codes into MFMA
// operands.  LDS: a 2-stage ring of activation and code tiles filled one step ahead by direct
// global->LDS loads (16-B pieces: 64-B runs of each weight row's codes), the tile rows' group
// sums (loaded once), and the weight rows' scales and biases in windows of 8 groups (one 16-B
// piece per row and window, double-buffered), so small per-group values do not cost a cache
// line request per row and step.
#include "common.h"
#include "gemm_dev.h"
#include "kernels.h"

#include <algorithm>
#include <type_traits>

namespace astro {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int XQ_W = 8;                          // waves per workgroup
constexpr int XQ_NT = 64 * XQ_W;                 // weight rows per tile
constexpr int XQ_KS = 128;                       // K per step
constexpr int XQ_OA = 0;                         // activations: 64 rows x 256 B
constexpr int XQ_OC = XQ_OA + 64 * 256;          // codes: 512 rows x 64 B
constexpr int XQ_SLOT = XQ_OC + XQ_NT * 64;      // 48 KB per ring stage
constexpr int XQ_OX = 2 * XQ_SLOT;               // group sums: 64 rows x G floats (G <= 64)
constexpr int XQ_OW = XQ_OX + 64 * 64 * 4;       // scale / bias windows: 2 x (512 x 16 B + 512 x 16 B)
constexpr int XQ_WIN = 2 * XQ_NT * 16;           // one window: scales, then biases
constexpr int kXqLds = XQ_OW + 2 * XQ_WIN;       // 144 KB

__device__ __forceinline__ int xq_aswz(int r) { return r & 15; }        // 16-B chunk XOR of a 256-B activation row
__device__ __forceinline__ int xq_cswz(int t) { return (t >> 2) & 3; }  // 16-B piece XOR of a 64-B code row

// inputs (0, 4), (1, 5), (2, 6), (3, 7) of 8 consecutive bf16 values: the codes' pairing
__device__ __forceinline__ u32x4 xq_pair(const u32x4 &d) {
  u32x4 a;
  a[0] = (d[0] & 0xffffu) | (d[2] << 16);
  a[1] = (d[0] >> 16) | (d[2] & 0xffff0000u);
  a[2] = (d[1] & 0xffffu) | (d[3] << 16);
  a[3] = (d[1] >> 16) | (d[3] & 0xffff0000u);
  return a;
}

// EPI: epilogue; GS: 32-input steps per group (1, 2, 4); PAIRED: the activation rows are stored
// in the codes' pairing.
template <int EPI, int GS, bool PAIRED>
__global__ __launch_bounds__(64 * XQ_W) void xq_gemm_kernel(const GemmArgs pa, const GemmArgs pb, int split, int nba,
                                                            int nbb) {
  extern __shared__ __attribute__((aligned(16))) char xq_lds[];
  int bx, by;
  tile_of_block(bx, by);
  const bool second = bx >= split;
  const GemmArgs p = second ? pb : pa;
  int expert, row0, m_valid;
  if (!gemm_tile(p, bx, by, second, split, second ? nbb : nba, expert, row0, m_valid)) return;
  const int nblk = by;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nk = p.K / XQ_KS;
  const int G = p.K / p.group;         // groups per row (a multiple of 8)
  constexpr int SPW = 2 * GS;          // steps per window of 8 groups (8 g / 128)

  // weight row of tile row t (SwiGLU: wave t / 64's 32 columns, gate rows then up rows)
  auto weight_row = [&](int t, bool &upper) {
    int n;
    if (EPI == kEpiSwiglu) {
      const int u = t & 63;
      upper = u >= 32;
      n = nblk * (XQ_NT / 2) + (t >> 6) * 32 + (u & 31);
    } else {
      upper = false;
      n = nblk * XQ_NT + t;
    }
    return n < p.N ? n : p.N - 1;  // rows past N load a valid row; never stored
  };
  // activation source row of tile row r (rows past m_valid read the tile's first row)
  auto source_row = [&](int r) {
    int src = row0 + (r < m_valid ? r : 0);
    if (p.a_rows) src = (int)(p.a_rows[src] / (uint32_t)p.a_div);
    if (p.a_rows2) src = (int)p.a_rows2[src];
    return src;
  };

  // ---- this lane's sources of the ring loads: 2 activation pieces, 4 code pieces per step
  const uint16_t *asrc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = (2 * wave + i) * 64 + lane, r = q >> 4, pc = q & 15;
    asrc[i] = p.A + (int64_t)source_row(r) * p.lda + 8 * (pc ^ xq_aswz(r));
  }
  const uint32_t *csrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = (4 * wave + i) * 64 + lane, t = q >> 2, pc = q & 3;
    bool up;
    const int n = weight_row(t, up);
    csrc[i] = (up ? p.w1 : p.w0) + (int64_t)expert * p.w_expert_stride + (int64_t)n * p.w_row_stride +
              4 * (pc ^ xq_cswz(t));
  }
  // scale / bias windows: this lane's weight row 64 w + lane
  const uint16_t *ssrc, *bsrc;
  {
    bool up;
    const int n = weight_row(64 * wave + lane, up);
    const int64_t so = (int64_t)expert * p.sb_expert_stride + (int64_t)n * p.sb_row_stride;
    ssrc = (up ? p.s1 : p.s0) + so;
    bsrc = (up ? p.b1 : p.b0) + so;
  }

  auto issue_step = [&](int k) {
    const int k0 = k * XQ_KS;
    char *slot = xq_lds + (k & 1) * XQ_SLOT;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds((const void *)(asrc[i] + k0), (lds_void *)(slot + XQ_OA + (2 * wave + i) * 1024),
                                       16, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((const void *)(csrc[i] + k0 / 8), (lds_void *)(slot + XQ_OC + (4 * wave + i) * 1024),
                                       16, 0, 0);
  };
  auto issue_window = [&](int v) {  // groups 8 v .. 8 v + 7 of every weight row
    char *win = xq_lds + XQ_OW + (v & 1) * XQ_WIN;
    __builtin_amdgcn_global_load_lds((const void *)(ssrc + 8 * v), (lds_void *)(win + wave * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void *)(bsrc + 8 * v), (lds_void *)(win + XQ_NT * 16 + wave * 1024), 16,
                                     0, 0);
  };
  // the tile rows' group sums, once: row r's G floats at XQ_OX + r * 4 G
  {
    const int ppr = G / 4, total = 64 * ppr;  // 16-B pieces per row, in all
    for (int q0 = 0; q0 < total; q0 += 64 * XQ_W) {
      const int q = q0 + wave * 64 + lane;
      if (q < total) {
        const int r = q / ppr, pc = q - r * ppr;
        __builtin_amdgcn_global_load_lds((const void *)(p.xsum + (int64_t)source_row(r) * p.xsum_ld + 4 * pc),
                                         (lds_void *)(xq_lds + XQ_OX + (q0 + wave * 64) * 16), 16, 0, 0);
      }
    }
  }
  issue_window(0);
  issue_step(0);

  const int c16 = lane & 15, kq = lane >> 4;
  const int nrb = (m_valid + 15) >> 4;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[4][4], part[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      acc[rb][nb] = zero;
      part[rb][nb] = zero;
    }

  auto consume = [&](auto nr_tag) {
    constexpr int NR = decltype(nr_tag)::value;  // row blocks computed
    for (int k = 0; k < nk; ++k) {
      __builtin_amdgcn_s_waitcnt(0x0f70);  // this wave's loads of step k (and its window)
      ring_barrier();                      // every wave's; every wave is done with step k - 1
      if (k + 1 < nk) {
        if ((k + 1) % SPW == 0) issue_window((k + 1) / SPW);
        issue_step(k + 1);
      }
      const char *slot = xq_lds + (k & 1) * XQ_SLOT;
      const char *win = xq_lds + XQ_OW + ((k / SPW) & 1) * XQ_WIN;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // B: the wave's four 16-row blocks, inputs 32 j + 8 kq .. +8 as (128 + q) pairs (i, i + 4)
        u32x4 bq[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const int t = 64 * wave + 16 * nb + c16;
          const uint32_t wd = *(const uint32_t *)(slot + XQ_OC + t * 64 + 16 * (j ^ xq_cswz(t)) + 4 * kq);
          bq[nb][0] = (wd & 0x000f000fu) | 0x43004300u;
          bq[nb][1] = ((wd >> 4) & 0x000f000fu) | 0x43004300u;
          bq[nb][2] = ((wd >> 8) & 0x000f000fu) | 0x43004300u;
          bq[nb][3] = ((wd >> 12) & 0x000f000fu) | 0x43004300u;
        }
        u32x4 af[NR];
#pragma unroll
        for (int rb = 0; rb < NR; ++rb) {
          const int r = 16 * rb + c16;
          const u32x4 d = *(const u32x4 *)(slot + XQ_OA + r * 256 + 16 * ((4 * j + kq) ^ xq_aswz(r)));
          af[rb] = PAIRED ? d : xq_pair(d);
        }
        // the first 32-input step of a group starts its partials afresh
        constexpr bool fresh_always = GS == 1;
        const bool fresh = fresh_always || j % GS == 0;
#pragma unroll
        for (int rb = 0; rb < NR; ++rb)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb)
            part[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[rb]),
                                                                   __builtin_bit_cast(bf16x8, bq[nb]),
                                                                   fresh ? zero : part[rb][nb], 0, 0, 0);
        // the group ends with this 32-input step: acc += s P + (b - 128 s) X
        if ((j + 1) % GS == 0) {
          const int gg = (k * XQ_KS + 32 * (j + 1)) / (32 * GS) - 1;  // the group
          const int gw = gg & 7;                                     // its place in the window
          float sv[4], cv[4];
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) {
            const int t = 64 * wave + 16 * nb + c16;
            const float s = bf2f(*(const uint16_t *)(win + t * 16 + 2 * gw));
            sv[nb] = s;
            cv[nb] = __builtin_fmaf(-128.0f, s, bf2f(*(const uint16_t *)(win + XQ_NT * 16 + t * 16 + 2 * gw)));
          }
#pragma unroll
          for (int rb = 0; rb < NR; ++rb) {
            float xs[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              xs[i] = *(const float *)(xq_lds + XQ_OX + (16 * rb + 4 * kq + i) * (4 * G) + 4 * gg);
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                acc[rb][nb][i] = __builtin_fmaf(cv[nb], xs[i], __builtin_fmaf(sv[nb], part[rb][nb][i], acc[rb][nb][i]));
          }
        }
      }
    }
  };
  if (nrb <= 1) consume(std::integral_constant<int, 1>());
  else if (nrb <= 2) consume(std::integral_constant<int, 2>());
  else if (nrb <= 3) consume(std::integral_constant<int, 3>());
  else consume(std::integral_constant<int, 4>());

  // ---- epilogue: lane holds column c16 of each block, rows 4 kq + i
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    if (rb >= nrb) break;
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
      uint16_t *crow = p.C + (int64_t)dsts[i] * p.ldc;
      if (EPI == kEpiSwiglu) {
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const int col = nblk * (XQ_NT / 2) + wave * 32 + f * 16 + c16;
          if (col < p.N) crow[col] = (uint16_t)swiglu_bf(round_bf(acc[rb][f][i]), round_bf(acc[rb][f + 2][i]));
        }
      } else {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const int col = nblk * XQ_NT + wave * 64 + nb * 16 + c16;
          if (col < p.N) {
            float v = acc[rb][nb][i];
            if (EPI == kEpiBias) v = round_bf(v) + bf2f(p.bias[col]);
            crow[col] = (uint16_t)f2bf(v);
          }
        }
      }
    }
  }
}

// X[r][gi] = the fp32 sum of inputs gi * g .. + g of row r (in input order): the group sums of
// the exact-code GEMM's affine terms; with paired set, also the row in the codes' pairing
// (inputs (0, 4), (1, 5), (2, 6), (3, 7) of every 8).  One thread per (row, group).
__global__ __launch_bounds__(256) void group_sums_kernel(const uint16_t *__restrict__ A, int64_t lda, int rows, int K,
                                                         int g, float *__restrict__ X, int64_t ldx,
                                                         uint16_t *__restrict__ paired) {
  const int G = K / g;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * G) return;
  const int r = (int)(i / G), gi = (int)(i - (int64_t)r * G);
  const u32x4 *src = (const u32x4 *)(A + (int64_t)r * lda + (int64_t)gi * g);
  u32x4 *dst = paired ? (u32x4 *)(paired + (int64_t)r * K + (int64_t)gi * g) : nullptr;
  float sum = 0.0f;
  for (int c = 0; c < g / 8; ++c) {
    const u32x4 v = src[c];
#pragma unroll
    for (int w = 0; w < 4; ++w) sum = (sum + bf_lo(v[w])) + bf_hi(v[w]);
    if (dst) dst[c] = xq_pair(v);
  }
  X[(int64_t)r * ldx + gi] = sum;
}

}  // namespace

bool xq_supported(const GemmArgs &a) {
  // 4-bit weights, K steps of 128, groups of 32 / 64 / 128 with a multiple of 8 of them per row
  // (16-B windows of scales), the activation rows' group sums at hand, 16-B aligned rows
  if (a.bkind != kBQ4 || !a.xsum || a.K % XQ_KS != 0) return false;
  if (a.group != 32 && a.group != 64 && a.group != 128) return false;
  const int G = a.K / a.group;
  return G % 8 == 0 && G <= 64 && a.lda % 8 == 0 && a.w_row_stride % 4 == 0 && a.sb_row_stride % 8 == 0 &&
         a.sb_expert_stride % 8 == 0 && a.xsum_ld % 4 == 0;
}

hipError_t launch_xq(const GemmArgs &a, const GemmArgs *b, int epi, hipStream_t s) {
  auto shape = [&](const GemmArgs &g, int &mt, int &nb) {
    nb = epi == kEpiSwiglu ? (g.N + XQ_NT / 2 - 1) / (XQ_NT / 2) : (g.N + XQ_NT - 1) / XQ_NT;
    mt = g.tile_expert ? g.max_tiles : (g.M + BM - 1) / BM;
    mt = mt > 0 && nb > 0 ? (mt + 7) & ~7 : 0;  // one XCD per row tile (see launch_kind)
  };
  int mta, nba, mtb = 0, nbb = 0;
  shape(a, mta, nba);
  if (b) shape(*b, mtb, nbb);
  if (mta + mtb == 0) return hipSuccess;
  const GemmArgs &bb = b ? *b : a;
  dim3 grid(mta + mtb, std::max(nba, nbb)), block(64 * XQ_W);
  auto launch = [&](auto kernel) {
    // > 64 KB of LDS is an opt-in per kernel (idempotent; cheap next to the launch)
    const hipError_t e = hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kXqLds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, grid, block, kXqLds, s, a, bb, mta, nba, nbb);
    return hipGetLastError();
  };
  auto by_group = [&](auto epi_tag, auto paired_tag) {
    constexpr int E = decltype(epi_tag)::value;
    constexpr bool P = decltype(paired_tag)::value;
    if (a.group == 32) return launch(xq_gemm_kernel<E, 1, P>);
    if (a.group == 64) return launch(xq_gemm_kernel<E, 2, P>);
    return launch(xq_gemm_kernel<E, 4, P>);
  };
  auto by_epi = [&](auto paired_tag) {
    if (epi == kEpiSwiglu) return by_group(std::integral_constant<int, kEpiSwiglu>(), paired_tag);
    if (epi == kEpiBias) return by_group(std::integral_constant<int, kEpiBias>(), paired_tag);
    return by_group(std::integral_constant<int, kEpiPlain>(), paired_tag);
  };
  if (a.a_paired) return by_epi(std::true_type());
  return by_epi(std::false_type());
}

hipError_t launch_group_sums(const uint16_t *A, int64_t lda, int rows, int K, int group, float *X, int64_t ldx,
                             uint16_t *paired, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const int64_t n = (int64_t)rows * (K / group);
  hipLaunchKernelGGL(group_sums_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, A, lda, rows, K, group,
                     X, ldx, paired);
  return hipGetLastError();
}

}  // namespace astro
