// Per-token routing on one wave (routing.rs:16-48), shared by the standalone route
// kernel and the decode path so both produce identical bits.
#pragma once

#include "common.h"

namespace astro {

// Lane j holds experts j, j+64, ...; softmax denominator = each lane's sequential sum,
// then the 64-lane tree (wave_sum); p = bf16(e * (1/S)).
//
// Top-k keys are (bf16(p) << 16 | expert) + 1 (0 marks an empty entry): a larger key is a
// larger probability with ties broken toward the higher expert index, as MLX's (value,
// index) partition comparator orders them.  Each lane keeps its PER keys sorted
// descending; k rounds of a wave-wide maximum over the lanes' heads (DPP, one readlane)
// take the keys in descending order and the winning lane pops its head.  Round r fills
// slot k-1-r, so lane j < k ends with slot j of the ascending slice and returns its expert
// and (renormalised) score as bf16 bits.  The renormalisation sums the slice in slot order
// from LDS.
// PER = experts per lane (ceil(E / 64), E <= 64 * PER); KMAX >= k, a multiple of 4;
// sh = KMAX words of LDS owned by this wave, 16-byte aligned.
template <int PER, int KMAX>
__device__ __forceinline__ void route_token(const uint16_t *__restrict__ l, int E, int k,
                                            int normalize, uint32_t *sh, uint32_t &out_idx,
                                            uint32_t &out_score) {
#pragma clang fp contract(off)
  const int lane = (int)(threadIdx.x & 63);
  float v[PER];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    // every load issued unconditionally (lanes past E read expert E-1 and drop it)
    const int e = lane + 64 * i;
    const float lv = bf2f(l[e < E ? e : E - 1]);
    v[i] = e < E ? lv : -__builtin_inff();
    m = fmaxf(m, v[i]);
  }
  m = wave_max_bcast(m);
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const float ex = det_expf(v[i] - m);
    v[i] = e < E ? ex : 0.0f;
    part = part + v[i];
  }
  const float rcp = 1.0f / wave_sum(part);
  uint32_t cand[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const uint32_t key = ((f2bf(v[i] * rcp) << 16) | (uint32_t)e) + 1u;
    cand[i] = e < E ? key : 0u;
  }
  // per-lane descending order (odd-even transposition network)
#pragma unroll
  for (int pass = 0; pass < PER; ++pass)
#pragma unroll
    for (int i = pass & 1; i + 1 < PER; i += 2) {
      const uint32_t hi = max(cand[i], cand[i + 1]), lo = min(cand[i], cand[i + 1]);
      cand[i] = hi;
      cand[i + 1] = lo;
    }
  uint32_t my_key = 0;
  for (int r = 0; r < k; ++r) {
    const uint32_t top = wave_max_u32_bcast(cand[0]);
    const bool hit = cand[0] == top;
#pragma unroll
    for (int i = 0; i + 1 < PER; ++i) cand[i] = hit ? cand[i + 1] : cand[i];
    cand[PER - 1] = hit ? 0u : cand[PER - 1];
    my_key = lane == k - 1 - r ? top - 1u : my_key;
  }
  const uint32_t sorted_key = my_key;
  float s = bf2f(sorted_key >> 16);
  if (normalize) {
    // sum over the slice in slot order
    if (lane < k) sh[lane] = __float_as_uint(s);
    __builtin_amdgcn_wave_barrier();
    u32x4 kv[KMAX / 4];
#pragma unroll
    for (int j = 0; j < KMAX / 4; ++j) kv[j] = ((const u32x4 *)sh)[j];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      const float nxt = sum + __uint_as_float(kv[j / 4][j % 4]);
      sum = j < k ? nxt : sum;
    }
    s = s / round_bf(sum);
  }
  out_idx = sorted_key & 0xffffu;
  out_score = f2bf(s);
}

}  // namespace astro
