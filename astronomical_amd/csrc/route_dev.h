// Per-token routing on one wave (routing.rs:16-48), shared by the standalone route
// kernel and the decode path so both produce identical bits.
#pragma once

#include "common.h"

namespace astro {

constexpr int kRouteMaxPerLane = 16;  // experts per lane: E <= 1024

// Lane j holds experts j, j+64, ...; softmax denominator = each lane's sequential sum,
// then the 64-lane tree (wave_sum); p = bf16(e * (1/S)).  Top-k: k rounds of a wave-wide
// maximum over keys (bf16(p) << 16 | expert) — a larger key is a larger probability with
// ties broken toward the higher expert index, as MLX's (value, index) partition
// comparator orders them.  Slot k-1-r receives round r (ascending slice).  Lane j < k
// returns slot j's expert and (renormalised) score as bf16 bits.
__device__ __forceinline__ void route_token(const uint16_t *__restrict__ l, int E, int k,
                                            int normalize, uint32_t &out_idx,
                                            uint32_t &out_score) {
#pragma clang fp contract(off)
  const int lane = (int)(threadIdx.x & 63);
  const int per = (E + 63) >> 6;
  float v[kRouteMaxPerLane];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kRouteMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    v[i] = (i < per && e < E) ? bf2f(l[e]) : -__builtin_inff();
    m = fmaxf(m, v[i]);
  }
  m = wave_max(m);
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < kRouteMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    v[i] = (i < per && e < E) ? det_expf(v[i] - m) : 0.0f;
    part = part + v[i];
  }
  const float rcp = 1.0f / wave_sum(part);
  uint32_t cand[kRouteMaxPerLane];
#pragma unroll
  for (int i = 0; i < kRouteMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    // candidates are key + 1 so that 0 means "none / taken"
    cand[i] = (i < per && e < E) ? (((f2bf(v[i] * rcp) << 16) | (uint32_t)e) + 1u) : 0u;
  }
  uint32_t my_idx = 0, my_p = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t best = 0;
#pragma unroll
    for (int i = 0; i < kRouteMaxPerLane; ++i) best = cand[i] > best ? cand[i] : best;
    const uint32_t key = wave_max_u32(best) - 1u;
    const uint32_t e = key & 0xffffu;
    if ((int)(e & 63) == lane) {
#pragma unroll
      for (int i = 0; i < kRouteMaxPerLane; ++i)
        if (i == (int)(e >> 6)) cand[i] = 0u;
    }
    if (lane == k - 1 - r) {
      my_idx = e;
      my_p = key >> 16;
    }
  }
  float s = bf2f(my_p);
  if (normalize) {
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) sum = sum + __shfl(s, j, kWave);
    s = s / round_bf(sum);
  }
  out_idx = my_idx;
  out_score = f2bf(s);
}

}  // namespace astro
