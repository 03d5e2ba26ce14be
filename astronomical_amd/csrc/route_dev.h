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
// comparator orders them.  The k-th largest key is found by a radix select over the key
// bits with wave ballots; the k selected keys are compacted through `lds` (64 words per
// wave), ranked, and permuted so that lane j < k holds slot j of the ascending slice.
// Lane j < k returns slot j's expert and (renormalised) score as bf16 bits.
// PER = experts per lane (ceil(E / 64), E <= 64 * PER).
template <int PER>
__device__ __forceinline__ void route_token(const uint16_t *__restrict__ l, int E, int k,
                                            int normalize, uint32_t &out_idx,
                                            uint32_t &out_score, uint32_t *lds) {
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
  // radix select: thr = the k-th largest candidate (keys are distinct, so exactly k
  // candidates are >= thr); candidates stay below 2^30
  uint32_t thr = 0;
  for (int bit = 29; bit >= 0; --bit) {
    const uint32_t c = thr | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      cnt += __popcll(__ballot(cand[i] >= c));
    if (cnt >= k) thr = c;
  }
  // compact the selected keys into lds[0..k)
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int base = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const bool sel = cand[i] >= thr;
    const uint64_t mask = __ballot(sel);
    if (sel) lds[base + __popcll(mask & below)] = cand[i] - 1u;
    base += __popcll(mask);
  }
  __builtin_amdgcn_wave_barrier();
  // rank among the selected keys, then send each key to the lane of its rank
  const uint32_t key = lane < k ? lds[lane] : 0u;
  uint32_t rank = (uint32_t)lane;
  if (lane < k) {
    rank = 0;
    for (int j = 0; j < k; ++j) rank += lds[j] < key;
  }
  const uint32_t sorted_key = (uint32_t)__builtin_amdgcn_ds_permute((int)(rank * 4), (int)key);
  __builtin_amdgcn_wave_barrier();
  const uint32_t my_idx = sorted_key & 0xffffu;
  float s = bf2f(sorted_key >> 16);
  if (normalize) {
    // sum over the slice in slot order
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), j));
    s = s / round_bf(sum);
  }
  out_idx = my_idx;
  out_score = f2bf(s);
}

}  // namespace astro
