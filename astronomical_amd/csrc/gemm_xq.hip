// The exact-code grouped GEMM for 4-bit affine weights (and the activation rows' group sums
// it needs).  Built in its own object with MFMA results in VGPRs
// (-mllvm=-amdgpu-mfma-vgpr-form): the per-group affine terms are VALU work on the MFMA
// accumulators, which AGPRs would make cross the register files.
//
// No weight is dequantised.  A 32-input MFMA step never crosses an affine group, so a group's
// contribution to an output is
//   sum_k x (s q + b) = s * sum_k x (128 + q) + (b - 128 s) * sum_k x,
// the MFMA runs on the exact codes (128 + q is bf16 0x4300 | q: one AND-OR makes two of them)
// into a per-group fp32 partial P, folded at the group's end as acc += s P.  The second term,
// sum_g c[n][g] X[m][g] with c = b - 128 s and X the groups' sums of the activation row
// (GemmArgs::xsum), is itself a small product over the groups: fp32 MFMAs (16x16x4) add it four
// groups at a time.  The cheap unpack pairs the codes of inputs (i, i + 4) of each 8-input word,
// so the activation rows are stored in the same pairing (GemmArgs::a_paired: the copy of x
// group_sums_kernel writes, or the activated rows the SwiGLU epilogue writes).
//
// A workgroup of 8 waves (one per CU) owns a tile of up to kXqRows rows of one expert and 512
// weight rows (plain: 512 output columns; SwiGLU: 256 activated columns = 256 gate + 256 up
// rows), K stepped by 128.  Wave w owns weight rows 64 w .. +64 (SwiGLU: the gate rows, then
// the up rows, of 32 columns) and every 16-row block of the tile:
//   - its codes go from HBM straight into its registers: a step's register set, once unpacked,
//     takes the codes of the step two ahead (two register sets);
//     lane (column c, quarter q) of a 16-row block loads the words of its inputs per group,
//     and the MFMA's input order within the group follows that load (any order works when the
//     activation fragment uses the same one);
//   - the activation tile (gathered rows) goes through a 3-stage LDS ring filled by direct
//     global->LDS loads two steps ahead; one barrier per step;
//   - the scales and biases of the weight rows come in LDS windows of 8 groups (one 16-B piece
//     per row and window, double-buffered), the tile rows' group sums once per tile.
// A routed problem's tiles come from the sort's table (GemmArgs::xtiles): every expert's rows
// split into ceil(rows / kXqRows) tiles of balanced sizes, so no tile holds a small remainder.
// The SwiGLU epilogue can store the activated rows in the codes' pairing together with their
// group sums (GemmArgs::c_paired, c_xsum): the inputs of a following exact-code down projection.
#include "common.h"
#include "gemm_dev.h"
#include "kernels.h"

#include <algorithm>
#include <type_traits>

namespace astro {

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int XQ_NT = 512;                              // weight rows per tile
constexpr int XQ_NBW = 4;                               // 16-row blocks of weight rows per wave
constexpr int XQ_RW = 16 * XQ_NBW;                      // weight rows per wave
constexpr int XQ_W = XQ_NT / XQ_RW;                     // waves per workgroup
constexpr int XQ_KS = 128;                              // K per step
constexpr int XQ_MT = kXqRows;                          // rows per tile, at most
constexpr int XQ_NRMAX = XQ_MT / 16;                    // 16-row blocks per tile, at most
constexpr int XQ_STAGES = 3;                            // activation ring stages
constexpr int XQ_AR = 96;                               // activation rows loaded per stage (>= XQ_MT)
constexpr int XQ_ASTAGE = XQ_AR * 256;                  // one stage: XQ_AR rows x 256 B
constexpr int XQ_ALOADS = XQ_AR * 16 / (64 * XQ_W);     // 16-B pieces per lane and stage
static_assert(XQ_ALOADS * 64 * XQ_W == XQ_AR * 16, "whole activation pieces per lane");
static_assert(XQ_MT <= XQ_AR && XQ_MT % 16 == 0, "tile rows within the loaded rows");
constexpr int XQ_GMAX = 64;                             // groups per row, at most
constexpr int XQ_OX = XQ_STAGES * XQ_ASTAGE;            // group sums: XQ_MT rows x (G + 4) floats
constexpr int XQ_OW = XQ_OX + XQ_MT * (XQ_GMAX + 4) * 4;  // scale / bias windows
constexpr int XQ_WIN = 2 * XQ_NT * 16;                  // one window: scales, then biases
constexpr int kXqLds = XQ_OW + 2 * XQ_WIN;
static_assert(XQ_W * 64 == XQ_NT, "one weight row's window piece per lane");

// (128 + q) pairs of an 8-code word: inputs (0, 4), (1, 5), (2, 6), (3, 7), as four dwords.
// mask (0x000f000f, in an SGPR) and k43 (0x43004300, in a VGPR) are not constants to the
// compiler, so each dword is one v_and_or_b32 (a VOP3 takes no literal) with the compiler
// tracking the hazards of its result (inline asm would hide them from it).
__device__ __forceinline__ u32x4 xq_unpack(uint32_t w, uint32_t mask, uint32_t k43) {
  u32x4 r;
  r[0] = (w & mask) | k43;
  r[1] = ((w >> 4) & mask) | k43;
  r[2] = ((w >> 8) & mask) | k43;
  r[3] = ((w >> 12) & mask) | k43;
  return r;
}

// place of input e of an 8-input chunk in the codes' pairing (0 4 1 5 2 6 3 7)
__device__ __forceinline__ int xq_pair_pos(int col) { return (col & ~7) | ((col & 3) << 1) | ((col >> 2) & 1); }

// EPI: epilogue; GS: 32-input MFMA steps per group (1, 2, 4); NR: 16-row blocks computed;
// NBW: 16-row blocks of weight rows per wave: XQ_NBW for a whole tile, half of it for a half
// tile (weight rows half * NT .. + NT of the N-block's XQ_NT; SwiGLU: its activated columns
// half * NT / 2 .. + NT / 2).
template <int EPI, int GS, int NR, int NBW>
__device__ __forceinline__ void xq_tile(const GemmArgs &p, char *lds, int nblk, int half, int expert, int row0,
                                        int rows) {
  constexpr int RW = 16 * NBW;      // weight rows per wave
  constexpr int NT = XQ_W * RW;     // weight rows of the tile
  static_assert(NBW == XQ_NBW || NBW * 2 == XQ_NBW, "whole or half tiles");
  static_assert(EPI != kEpiSwiglu || NBW % 2 == 0, "a SwiGLU wave pairs its gate and up blocks");
  constexpr int NG = 4 / GS;        // groups per K step
  constexpr int NC = NBW * NG;      // code loads per lane and step (blocks x groups)
  constexpr int SPW = 8 / NG;       // K steps per window of 8 groups
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int nk = p.K / XQ_KS;
  const int G = p.K / p.group;
  const int xstride = (G + 4) * 4;  // bytes per row of the group sums (padded: no bank conflicts)

  // weight row of tile row t (SwiGLU: wave t / RW's RW / 2 columns, gate rows then up rows)
  auto weight_row = [&](int t, bool &upper) {
    int n;
    if (EPI == kEpiSwiglu) {
      const int u = t % RW;
      upper = u >= RW / 2;
      n = nblk * (XQ_NT / 2) + half * (NT / 2) + (t / RW) * (RW / 2) + u % (RW / 2);
    } else {
      upper = false;
      n = nblk * XQ_NT + half * NT + t;
    }
    return n < p.N ? n : p.N - 1;  // rows past N load a valid row; never stored
  };
  // activation source row of tile row r (rows past the tile's read its first row)
  auto source_row = [&](int r) {
    int src = row0 + (r < rows ? r : 0);
    if (p.a_rows) src = (int)(p.a_rows[src] / (uint32_t)p.a_div);
    if (p.a_rows2) src = (int)p.a_rows2[src];
    return src;
  };

  // ---- sources: this lane's activation pieces, code words and window row
  const uint16_t *asrc[XQ_ALOADS];
#pragma unroll
  for (int i = 0; i < XQ_ALOADS; ++i) {
    const int q = (XQ_ALOADS * wave + i) * 64 + lane, r = q >> 4, pc = q & 15;
    asrc[i] = p.A + (int64_t)source_row(r) * p.lda + 8 * (pc ^ (r & 15));
  }
  const uint32_t *csrc[NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    bool up;
    const int n = weight_row(RW * wave + 16 * nb + c16, up);
    csrc[nb] = (up ? p.w1 : p.w0) + (int64_t)expert * p.w_expert_stride + (int64_t)n * p.w_row_stride + GS * kq;
  }
  const uint16_t *ssrc, *bsrc;
  {
    bool up;
    // the window piece of tile row 64 wave + lane (a half tile's lanes past its NT rows load
    // its last row into window places nothing reads)
    const int n = weight_row(min(64 * wave + lane, NT - 1), up);
    const int64_t so = (int64_t)expert * p.sb_expert_stride + (int64_t)n * p.sb_row_stride;
    ssrc = (up ? p.s1 : p.s0) + so;
    bsrc = (up ? p.b1 : p.b0) + so;
  }

  uint32_t cw[2][NBW][4];  // code words: register set, 16-row block, word of the step
  auto issue_codes = [&](auto set_tag, int k) {
    constexpr int S = decltype(set_tag)::value;
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
      for (int h = 0; h < NG; ++h) {
        const uint32_t *src = csrc[nb] + k * 16 + h * 4 * GS;
        if (GS == 1) {
          cw[S][nb][h] = *src;
        } else if (GS == 2) {
          const u32x2 v = *(const u32x2 *)src;
          cw[S][nb][2 * h] = v[0];
          cw[S][nb][2 * h + 1] = v[1];
        } else {
          const u32x4 v = *(const u32x4 *)src;
#pragma unroll
          for (int j = 0; j < 4; ++j) cw[S][nb][j] = v[j];
        }
      }
  };
  auto issue_act = [&](int st, int k) {
    char *stage = lds + st * XQ_ASTAGE;
#pragma unroll
    for (int i = 0; i < XQ_ALOADS; ++i)
      __builtin_amdgcn_global_load_lds((const void *)(asrc[i] + k * XQ_KS),
                                       (lds_void *)(stage + (XQ_ALOADS * wave + i) * 1024), 16, 0, 0);
  };
  auto issue_window = [&](int v) {  // groups 8 v .. 8 v + 7 of every weight row
    char *win = lds + XQ_OW + (v & 1) * XQ_WIN;
    __builtin_amdgcn_global_load_lds((const void *)(ssrc + 8 * v), (lds_void *)(win + wave * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void *)(bsrc + 8 * v), (lds_void *)(win + XQ_NT * 16 + wave * 1024), 16,
                                     0, 0);
  };
  // the tile rows' group sums, once: row r's G floats at XQ_OX + r * xstride (16-B pieces; the
  // 4 pad floats of a row are not loaded)
  {
    const int ppr = G / 4 + 1, total = XQ_MT * ppr;  // pieces per padded row
    for (int q0 = wave * 64; q0 < total; q0 += 64 * XQ_W) {
      const int q = q0 + lane, r = q / ppr, pc = q - r * ppr;
      if (q < total && pc < G / 4)
        __builtin_amdgcn_global_load_lds((const void *)(p.xsum + (int64_t)source_row(r) * p.xsum_ld + 4 * pc),
                                         (lds_void *)(lds + XQ_OX + q0 * 16), 16, 0, 0);
    }
  }
  // every step issues the loads of the step two ahead (activations after the step's barrier,
  // codes once its own are unpacked), past the last step the last one again (into a stage and
  // register set nothing reads any more): the same count of loads per step keeps the waits
  // below exact
  issue_window(0);
  issue_act(0, 0);
  issue_codes(std::integral_constant<int, 0>(), 0);
  issue_act(1, min(1, nk - 1));
  issue_codes(std::integral_constant<int, 1>(), min(1, nk - 1));

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[NR][NBW];
#pragma unroll
  for (int rb = 0; rb < NR; ++rb)
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) acc[rb][nb] = zero;
  // opaque to the compiler (see xq_unpack): the mask in an SGPR, the exponent bits in a VGPR
  uint32_t mask = 0x000f000fu, k43 = 0x43004300u;
  asm volatile("" : "+s"(mask));
  asm volatile("" : "+v"(k43));

  // tail: the last step after the whole pairs.  The compiler drops the loads of its code words
  // nothing reads, so fewer loads than XQ_ALOADS + NC may follow its own: it waits for every load.
  auto step = [&](auto set_tag, int k, bool tail) {
    constexpr int S = decltype(set_tag)::value;  // register set: k % 2
    // this wave's loads of step k (issued two steps ago) are in; the next step's may not be
    if (tail) wait_vmcnt_le(0);
    else wait_vmcnt_le(XQ_ALOADS + NC);
    ring_barrier();  // every wave's loads of step k are in; every wave is done with step k - 1
    if (k % SPW == 0 && (k / SPW + 1) * 8 < G) issue_window(k / SPW + 1);
    const int ka = min(k + 2, nk - 1);
    const int st = k % 3;
    issue_act(st == 0 ? 2 : st - 1, ka);  // stage (k + 2) % 3: step k - 1's
    const char *stage = lds + st * XQ_ASTAGE;
    const char *win = lds + XQ_OW + ((k / SPW) & 1) * XQ_WIN;
#pragma unroll
    for (int h = 0; h < NG; ++h) {
      const int gg = k * NG + h;  // the group
      const int gw = gg & 7;      // its place in the window
      u32x4 bq[NBW][GS];
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
        for (int jj = 0; jj < GS; ++jj) bq[nb][jj] = xq_unpack(cw[S][nb][h * GS + jj], mask, k43);
      if (h == NG - 1) issue_codes(std::integral_constant<int, S>(), ka);  // this set is unpacked
      float sv[NBW];
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb)
        sv[nb] = bf2f(*(const uint16_t *)(win + (RW * wave + 16 * nb + c16) * 16 + 2 * gw));
      // per 16-row block, in issue order: the next block's activation fragments, the column
      // blocks' first MFMAs (independent), their next ones (each NBW MFMAs after the one it
      // depends on), then the folds of the previous block, whose MFMAs are done by then: the
      // VALU folds one block while the MFMA unit runs the next
      auto frags = [&](int rb, u32x4 *af) {
        const int r = 16 * rb + c16;
#pragma unroll
        for (int jj = 0; jj < GS; ++jj)
          af[jj] = *(const u32x4 *)(stage + r * 256 + 16 * ((4 * GS * h + GS * kq + jj) ^ (r & 15)));
      };
      auto mfmas = [&](const u32x4 *a, f32x4 *pp) {
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb)
          pp[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[0]),
                                                           __builtin_bit_cast(bf16x8, bq[nb][0]), zero, 0, 0, 0);
#pragma unroll
        for (int jj = 1; jj < GS; ++jj)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb)
            pp[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[jj]),
                                                             __builtin_bit_cast(bf16x8, bq[nb][jj]), pp[nb], 0, 0, 0);
      };
      auto fold = [&](int rb, const f32x4 *pp) {
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[rb][nb][i] = __builtin_fmaf(sv[nb], pp[nb][i], acc[rb][nb][i]);
      };
      u32x4 af[2][GS];
      f32x4 pp[2][NBW];
      frags(0, af[0]);
#pragma unroll
      for (int rb = 0; rb < NR; ++rb) {
        if (rb + 1 < NR) frags(rb + 1, af[(rb + 1) & 1]);
        mfmas(af[rb & 1], pp[rb & 1]);
        if (rb > 0) fold(rb - 1, pp[(rb - 1) & 1]);
      }
      fold(NR - 1, pp[(NR - 1) & 1]);
      // groups gg - 3 .. gg complete: acc += X[rows][4 groups] . c[4 groups][columns]
      if (gg % 4 == 3) {
        const int g4 = gg >> 2;
        const int gl = (4 * g4 + kq) & 7;  // this lane's group in the window
        float cq[NBW];
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
          const int t = RW * wave + 16 * nb + c16;
          const float s = bf2f(*(const uint16_t *)(win + t * 16 + 2 * gl));
          const float b = bf2f(*(const uint16_t *)(win + XQ_NT * 16 + t * 16 + 2 * gl));
          cq[nb] = __builtin_fmaf(-128.0f, s, b);
        }
#pragma unroll
        for (int rb = 0; rb < NR; ++rb) {
          const float xa = *(const float *)(lds + XQ_OX + (16 * rb + c16) * xstride + 4 * (4 * g4 + kq));
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb)
            acc[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, cq[nb], acc[rb][nb], 0, 0, 0);
        }
      }
    }
  };
  // whole pairs of steps, then the last one: on every path into a step the same loads follow
  // its codes, so the compiler's own waits for them stay partial
  int k0 = 0;
  for (; k0 + 2 <= nk; k0 += 2) {
    step(std::integral_constant<int, 0>(), k0, false);
    step(std::integral_constant<int, 1>(), k0 + 1, false);
  }
  if (k0 < nk) step(std::integral_constant<int, 0>(), k0, true);
  wait_vmcnt_le(0);  // the trailing repeated loads, before the ring is reused or the wave ends

  // ---- epilogue: lane holds column c16 of each block, rows 4 kq + i
  if (EPI == kEpiSwiglu) {
    const bool sums = p.c_xsum != nullptr;
    float rs[NR][4];
#pragma unroll
    for (int rb = 0; rb < NR; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rb * 16 + kq * 4 + i;
        const int gr = row0 + (r < rows ? r : 0);
        uint16_t *crow = p.C + (int64_t)(p.c_rows ? (int)p.c_rows[gr] : gr) * p.ldc;
        float s = 0.0f;
#pragma unroll
        for (int f = 0; f < NBW / 2; ++f) {
          const int col = nblk * (XQ_NT / 2) + half * (NT / 2) + wave * (RW / 2) + f * 16 + c16;
          const uint32_t a = swiglu_bf(round_bf(acc[rb][f][i]), round_bf(acc[rb][f + NBW / 2][i]));
          if (col < p.N) {
            if (r < rows) crow[p.c_paired ? xq_pair_pos(col) : col] = (uint16_t)a;
            s += bf2f(a);
          }
        }
        rs[rb][i] = s;
      }
    if (sums) {
      // the wave's RW / 2 columns of each row, then the waves of each group of c_group columns
#pragma unroll
      for (int rb = 0; rb < NR; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int o = 1; o < 16; o <<= 1) rs[rb][i] += __shfl_xor(rs[rb][i], o, 16);
      __syncthreads();  // every wave is done with the ring: its first stage holds the sums
      float *red = (float *)lds;  // [wave][XQ_MT]
      if (c16 == 0)
#pragma unroll
        for (int rb = 0; rb < NR; ++rb)
#pragma unroll
          for (int i = 0; i < 4; ++i) red[wave * XQ_MT + rb * 16 + kq * 4 + i] = rs[rb][i];
      __syncthreads();
      const int wpg = p.c_group / (RW / 2);  // waves per group
      const int gpt = XQ_W / wpg;               // groups of the tile
      const int g0 = (nblk * (XQ_NT / 2) + half * (NT / 2)) / p.c_group;
      const int ng = p.N / p.c_group;
      for (int q = tid; q < rows * gpt; q += 64 * XQ_W) {
        const int r = q / gpt, j = q - r * gpt;
        if (g0 + j >= ng) continue;
        float s = 0.0f;
        for (int w = 0; w < wpg; ++w) s += red[(j * wpg + w) * XQ_MT + r];
        const int gr = row0 + r;
        p.c_xsum[(int64_t)(p.c_rows ? (int)p.c_rows[gr] : gr) * p.c_xsum_ld + g0 + j] = s;
      }
    }
  } else {
    // The wave's rows x RW columns go through LDS (row-major, the ring's space, free once every
    // wave is past its last step) so that each lane stores 16-B pieces of a row: ten stores per
    // lane of whole 128-B lines instead of NR * NBW * 4 two-byte stores.  A tile reaching past
    // N, or an output that is not 16-B aligned, takes the element stores.
    const int col0 = nblk * XQ_NT + half * NT + wave * RW;
    // (the same for every wave of the workgroup: the barrier below is taken by all or none)
    const bool vec = p.ldc % 8 == 0 && ((uintptr_t)p.C & 15) == 0 && nblk * XQ_NT + half * NT + NT <= p.N;
    if (vec) {
      constexpr int OSTR = RW + 8;  // elements per staged row (16-B aligned rows)
      static_assert(XQ_W * XQ_MT * OSTR * 2 <= XQ_OW, "the staged outputs fit before the windows");
      __syncthreads();  // every wave is done reading the ring and the group sums
      uint16_t *ot = (uint16_t *)lds + wave * (XQ_MT * OSTR);
#pragma unroll
      for (int rb = 0; rb < NR; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb) {
            float v = acc[rb][nb][i];
            if (EPI == kEpiBias) v = round_bf(v) + bf2f(p.bias[col0 + nb * 16 + c16]);
            ot[(rb * 16 + kq * 4 + i) * OSTR + nb * 16 + c16] = (uint16_t)f2bf(v);
          }
      // the wave reads back its own writes: its LDS operations complete in order
      asm volatile("" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      constexpr int PR = RW / 8;  // 16-B pieces per row
      for (int q = lane; q < rows * PR; q += 64) {
        const int r = q / PR, c = q - r * PR;
        const u32x4 v = *(const u32x4 *)(ot + r * OSTR + 8 * c);
        uint16_t *crow = p.C + (int64_t)(p.c_rows ? (int)p.c_rows[row0 + r] : row0 + r) * p.ldc;
        *(u32x4 *)(crow + col0 + 8 * c) = v;
      }
    } else {
#pragma unroll
      for (int rb = 0; rb < NR; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = rb * 16 + kq * 4 + i;
          if (r >= rows) continue;
          uint16_t *crow = p.C + (int64_t)(p.c_rows ? (int)p.c_rows[row0 + r] : row0 + r) * p.ldc;
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb) {
            const int col = col0 + nb * 16 + c16;
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

// Workgroup -> tile.  The 8 XCDs take workgroups round-robin by index, and the dispatcher deals
// them strictly in order (a workgroup whose XCD has no free CU holds back the ones after it).
// The tiles are laid out per XCD: XCD j holds the row tiles x = j (mod 8) of both problems, each
// padded to a multiple of 8, the N-blocks of one row tile one after the other so they share its
// activation rows in that XCD's L2; the XCD's s-th workgroup takes place s (cx = 0: padded places
// return at once).
// With cx > 0 (the XCD's CUs) the real tiles past the XCD's last whole round of cx workgroups
// form a partial round; when it is at most half full, each of its tiles splits into two half
// tiles, the second half taken by the workgroups right after the XCD's real tiles (the grid has
// 8 cx extra workgroups for them), so the partial round takes about as long as a half tile.
// Then problem a's padding is skipped (its row count is known to the host: a has no tile
// table, or there is no b), b's real row tiles come first in its places, and both problems
// have nb N-blocks.  A workgroup's tile does not depend on the device-side tile count except for
// the second halves: its tile-table entry is loaded together with the count.  SPLIT: the kernel
// that splits (cx > 0); the other holds no half-tile code.
template <int EPI, int GS, bool SPLIT>
__global__ __launch_bounds__(64 * XQ_W) void xq_gemm_kernel(const GemmArgs pa, const GemmArgs pb, int split, int nba,
                                                            int nbb, int g0, int cx) {
  if (!SPLIT) cx = 0;
  extern __shared__ __attribute__((aligned(16))) char xq_lds[];
  const int nb = max(nba, nbb);
  const int l = (int)blockIdx.x;
  const int j = l & 7;                                   // the XCD
  const int S = g0 >> 3;                                 // the XCD's places in the padded layout
  const int pos = l < g0 ? l >> 3 : S + ((l - g0) >> 3);  // the workgroup's place in the XCD's sequence
  const int mt = g0 / nb;                                // padded row tiles of both problems
  const bool has_b = mt > split;
  const int qa = split >> 3;                             // a's padded row tiles per XCD
  // a's real row tiles on this XCD when a's padding is skipped (host-known row count)
  const int na = cx > 0 && has_b ? max(0, min(qa, ((pa.M + XQ_MT - 1) / XQ_MT - j + 7) >> 3)) : qa;
  // place t of the XCD's sequence (a's padding skipped) -> row tile bx, N-block by
  auto place = [&](int t, int &bx, int &by) {
    const int r = t / nb;
    by = t - r * nb;
    bx = 8 * (r < na ? r : qa + (r - na)) + j;
  };
  // a row tile's table entry (clamped into the table: a place past the real tiles loads a valid
  // entry that the count check then discards)
  // (fields picked by value: a reference to a kernel argument would copy both to scratch)
  auto entry = [&](int bx, uint32_t &e, uint32_t &r0) {
    const bool second = bx >= split;
    const uint32_t *xt = second ? pb.xtiles : pa.xtiles;
    if (xt) {
      const int x = min(second ? bx - split : bx, (second ? pb.max_xtiles : pa.max_xtiles) - 1);
      e = xt[2 + 2 * x];
      r0 = xt[3 + 2 * x];
    }
  };
  int bx, by, half = -1;  // half: -1 whole, 0 / 1 the halves of a split tile
  place(pos, bx, by);
  uint32_t e = 0, r0 = 0;
  entry(bx, e, r0);
  const int cnt_a = pa.xtiles ? (int)pa.xtiles[0] : (pa.M + XQ_MT - 1) / XQ_MT;
  const int cnt_b = has_b ? (pb.xtiles ? (int)pb.xtiles[0] : (pb.M + XQ_MT - 1) / XQ_MT) : 0;
  if (cx > 0) {
    // the XCD's real tiles
    const int f = nb * (max(0, min(qa, (cnt_a - j + 7) >> 3)) + max(0, min((mt - split) >> 3, (cnt_b - j + 7) >> 3)));
    int tail0 = f / cx * cx, tail = f - tail0;
    if (2 * tail > cx) tail0 = f, tail = 0;  // more than half a round: splitting would not shorten it
    if (pos >= f) {
      if (pos - f >= tail) return;
      place(tail0 + (pos - f), bx, by);
      entry(bx, e, r0);
      half = 1;
    } else if (pos >= tail0) {
      half = 0;
    }
  }
  const bool second = bx >= split;
  const GemmArgs p = second ? pb : pa;
  if (by >= (second ? nbb : nba)) return;
  const int x = second ? bx - split : bx;
  if (x >= (second ? cnt_b : cnt_a)) return;
  int expert = 0, row0, rows;
  if (p.xtiles) {
    expert = (int)(e & 0xffffu);
    rows = (int)(e >> 16);
    row0 = (int)r0;
  } else {
    row0 = x * XQ_MT;
    rows = min(XQ_MT, p.M - row0);
  }
  if (rows <= 0) return;
  const int nr = (rows + 15) >> 4;
  auto dispatch = [&](auto nbw_tag, int h) {
    constexpr int W = decltype(nbw_tag)::value;
    if (nr <= 1) xq_tile<EPI, GS, 1, W>(p, xq_lds, by, h, expert, row0, rows);
    else if (nr == 2) xq_tile<EPI, GS, 2, W>(p, xq_lds, by, h, expert, row0, rows);
    else if (nr == 3) xq_tile<EPI, GS, 3, W>(p, xq_lds, by, h, expert, row0, rows);
    else if (XQ_NRMAX == 4 || nr == 4) xq_tile<EPI, GS, 4, W>(p, xq_lds, by, h, expert, row0, rows);
    else if (XQ_NRMAX == 5 || nr == 5) xq_tile<EPI, GS, (XQ_NRMAX < 5 ? 4 : 5), W>(p, xq_lds, by, h, expert, row0, rows);
    else xq_tile<EPI, GS, XQ_NRMAX, W>(p, xq_lds, by, h, expert, row0, rows);
  };
  static_assert(XQ_NRMAX >= 4 && XQ_NRMAX <= 6, "tiles of 64 to 96 rows");
  if (!SPLIT || half < 0) dispatch(std::integral_constant<int, XQ_NBW>(), 0);
  else dispatch(std::integral_constant<int, XQ_NBW / 2>(), half);
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
  X[(int64_t)r * ldx + gi] = group_sum_paired(src, g, dst);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

bool xq_supported(const GemmArgs &a) {
  // 4-bit weights, K steps of 128, groups of 32 / 64 / 128 with a multiple of 8 of them per row
  // (16-B windows of scales), the activation rows paired and their group sums at hand, 16-B
  // aligned rows
  if (a.bkind != kBQ4 || !a.xsum || !a.a_paired || a.K % XQ_KS != 0) return false;
  // (groups of 128 need more registers than the tile leaves: the dequantising kernels take them)
  if (a.group != 32 && a.group != 64) return false;
  const int G = a.K / a.group;
  if (G % 8 != 0 || G > XQ_GMAX) return false;
  if (a.lda % 8 || a.w_row_stride % 4 || a.sb_row_stride % 8 || a.sb_expert_stride % 8 || a.xsum_ld % 4 ||
      a.w_expert_stride % 4)
    return false;
  if (!aligned16(a.A) || !aligned16(a.w0) || !aligned16(a.s0) || !aligned16(a.b0) || !aligned16(a.xsum)) return false;
  if (a.w1 && (!aligned16(a.w1) || !aligned16(a.s1) || !aligned16(a.b1))) return false;
  // the epilogue's pairing and group sums: whole groups of 32 / 64 / 128 activated columns
  if (a.c_xsum && (a.c_group % (XQ_RW / 2) || a.c_group > 128 || a.N % a.c_group)) return false;
  return true;
}

static int xq_max_tiles(const GemmArgs &a) {
  return a.xtiles ? a.max_xtiles : (a.M + XQ_MT - 1) / XQ_MT;
}

// CUs per XCD of the current device (its 8 XCDs take workgroups round-robin); 0 if unknown
static int xq_cus_per_xcd() {
  static int cached[64];  // per device; written once with the same value by any thread
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) return 0;
    cached[dev] = n / 8;
  }
  return cached[dev];
}

hipError_t launch_xq(const GemmArgs &a, const GemmArgs *b, int epi, hipStream_t s) {
  auto shape = [&](const GemmArgs &g, int &mt, int &nb) {
    nb = epi == kEpiSwiglu ? (g.N + XQ_NT / 2 - 1) / (XQ_NT / 2) : (g.N + XQ_NT - 1) / XQ_NT;
    mt = xq_max_tiles(g);
    mt = mt > 0 && nb > 0 ? (mt + 7) & ~7 : 0;  // one XCD per row tile
  };
  int mta, nba, mtb = 0, nbb = 0;
  shape(a, mta, nba);
  if (b) shape(*b, mtb, nbb);
  if (mta + mtb == 0) return hipSuccess;
  const GemmArgs &bb = b ? *b : a;
  const int nb = std::max(nba, nbb), g0 = (mta + mtb) * nb;
  // half tiles of a partial last round: K long enough that a tile's time is mostly its K steps
  // (a half tile of a few steps takes nearly as long as a whole one), both problems with the
  // same N-blocks, problem a's row count known here when there is a b (no tile table), and a
  // half tile's activated columns (XQ_NT / 4) whole groups of the epilogue's sums
  int cx = a.K / XQ_KS >= 8 ? xq_cus_per_xcd() : 0;
  if ((mtb > 0 && (nba != nbb || a.xtiles)) || (epi == kEpiSwiglu && a.c_xsum && (XQ_NT / 4) % a.c_group) ||
      (epi == kEpiSwiglu && mtb > 0 && bb.c_xsum && (XQ_NT / 4) % bb.c_group))
    cx = 0;
  dim3 grid(g0 + 8 * cx), block(64 * XQ_W);
  auto launch = [&](auto kernel) {
    // > 64 KB of LDS is an opt-in per kernel (idempotent; cheap next to the launch)
    const hipError_t e = hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kXqLds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, grid, block, kXqLds, s, a, bb, mta, nba, nbb, g0, cx);
    return hipGetLastError();
  };
  auto by_group = [&](auto epi_tag) {
    constexpr int E = decltype(epi_tag)::value;
    if (cx > 0) return a.group == 32 ? launch(xq_gemm_kernel<E, 1, true>) : launch(xq_gemm_kernel<E, 2, true>);
    return a.group == 32 ? launch(xq_gemm_kernel<E, 1, false>) : launch(xq_gemm_kernel<E, 2, false>);
  };
  if (epi == kEpiSwiglu) return by_group(std::integral_constant<int, kEpiSwiglu>());
  if (epi == kEpiBias) return by_group(std::integral_constant<int, kEpiBias>());
  return by_group(std::integral_constant<int, kEpiPlain>());
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
