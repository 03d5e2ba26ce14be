// Per-token routing on one wave (routing.rs:16-48), shared by the standalone route
// kernel and the decode path so both produce identical bits.
#pragma once

#include "common.h"

namespace astro {

// Lane j holds experts j, j+64, ...; softmax denominator = each lane's sequential sum,
// then the 64-lane tree (wave_sum); p = bf16(e * (1/S)).
//
// Top-k keys are (bf16(p) << 16 | expert): a larger key is a larger probability with
// ties broken toward the higher expert index, as MLX's (value, index) partition
// comparator orders them.  k rounds of a wave-wide maximum (DPP) take the keys in
// descending order; lane j < k keeps slot j of the ascending slice and returns its
// expert and (renormalised) score as bf16 bits.
// PER = experts per lane (ceil(E / 64), E <= 64 * PER).
template <int PER>
__device__ __forceinline__ void route_token(const uint16_t *__restrict__ l, int E, int k,
                                            int normalize, uint32_t &out_idx,
                                            uint32_t &out_score) {
#pragma clang fp contract(off)
  const int lane = (int)(threadIdx.x & 63);
  float v[PER];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    v[i] = (e < E) ? bf2f(l[e]) : -__builtin_inff();
    m = fmaxf(m, v[i]);
  }
  m = wave_max_fast(m);
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    v[i] = (e < E) ? det_expf(v[i] - m) : 0.0f;
    part = part + v[i];
  }
  const float rcp = 1.0f / wave_sum(part);
  uint32_t cand[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    // key + 1, so that 0 marks an empty entry
    cand[i] = (e < E) ? (((f2bf(v[i] * rcp) << 16) | (uint32_t)e) + 1u) : 0u;
  }
  // k rounds of a wave-wide maximum; round r fills slot k-1-r (ascending slice)
  uint32_t my_key = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t best = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) best = max(best, cand[i]);
    const uint32_t top = wave_max_u32_fast(best);
#pragma unroll
    for (int i = 0; i < PER; ++i) cand[i] = cand[i] == top ? 0u : cand[i];
    my_key = lane == k - 1 - r ? top - 1u : my_key;
  }
  const uint32_t sorted_key = my_key;
  float s = bf2f(sorted_key >> 16);
  if (normalize) {
    // sum over the slice in slot order
    float sum = 0.0f;
    for (int j = 0; j < k; ++j)
      sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), j));
    s = s / round_bf(sum);
  }
  out_idx = sorted_key & 0xffffu;
  out_score = f2bf(s);
}

}  // namespace astro
