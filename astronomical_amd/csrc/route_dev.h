// Per-token routing on one wave (routing.rs:16-48), shared by the standalone route
// kernel and the decode path so both produce identical bits.
#pragma once

#include "common.h"

namespace astro {

// Softmax of one token's logits (precise: fp32 inside, p rounded to bf16).  Lane j holds
// experts j, j+64, ... (PER of them, E <= 64 * PER); the denominator is each lane's
// sequential sum, then the 64-lane tree (wave_sum); p = bf16(e * (1/S)).  pbits[i] is the
// bf16 pattern of expert lane + 64 i (0 past E).
template <int PER>
__device__ __forceinline__ void route_probabilities(const uint16_t *__restrict__ l, int E, uint32_t (&pbits)[PER]) {
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
#pragma unroll
  for (int i = 0; i < PER; ++i) pbits[i] = lane + 64 * i < E ? f2bf(v[i] * rcp) : 0u;
}

// Scores of the slice: lane j < k holds its slot's bf16 probability; the renormalisation
// divides by the slice's sum in slot order (fp32, rounded to bf16) from LDS.  sh = KMAX words
// of this wave's LDS, 16-byte aligned.
template <int KMAX>
__device__ __forceinline__ uint32_t route_scores(uint32_t pbits, int k, int normalize, uint32_t *sh) {
#pragma clang fp contract(off)
  const int lane = (int)(threadIdx.x & 63);
  float s = bf2f(pbits);
  if (normalize) {
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
  return f2bf(s);
}

// The top-k SET of one token, fast: keys (bf16(p) << 16 | expert) + 1 (0 marks an empty
// entry), so a larger key is a larger probability with ties toward the higher expert index,
// the order of MLX's (value, index) partition comparator.  Each lane keeps its PER keys
// sorted descending; k rounds of a wave-wide maximum over the lanes' heads (DPP, one
// readlane) take the keys in descending order and the winning lane pops its head.  Round r
// fills slot k-1-r, so lane j < k ends with slot j of the slice in ascending key order and
// returns its expert and (renormalised over that order) score.  The set equals
// route_token_exact's; the order within it does not (callers that need only the set use this).
// PER = experts per lane (ceil(E / 64)); KMAX >= k, a multiple of 4; sh = KMAX words of LDS
// owned by this wave, 16-byte aligned.
template <int PER, int KMAX>
__device__ __forceinline__ void route_token(const uint16_t *__restrict__ l, int E, int k,
                                            int normalize, uint32_t *sh, uint32_t &out_idx,
                                            uint32_t &out_score) {
  const int lane = (int)(threadIdx.x & 63);
  uint32_t pb[PER];
  route_probabilities<PER>(l, E, pb);
  uint32_t cand[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    cand[i] = e < E ? ((pb[i] << 16) | (uint32_t)e) + 1u : 0u;
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
  out_idx = my_key & 0xffffu;
  out_score = route_scores<KMAX>(my_key >> 16, k, normalize, sh);
}

// The 8 largest keys of a wave, descending, in every lane (uniform values): each lane's list of
// its 8 largest keys (descending; 0 pads), then six bitonic merges with a partner lane's list
// fetched by DPP -- lane ^ 1, lane ^ 2 (quads), row rotations by 4 and 8 (rows), then row 15's
// list into rows 1 and 3 and row 31's into rows 2 and 3 -- after which lane 63 holds the wave's
// 8 largest.  A merge keeps the top 8 of two descending lists a, b: c_i = max(a_i, b_{7-i}) is a
// bitonic sequence holding them, sorted by three half-cleaner stages.  Partner lists are
// disjoint at every level (rows not written by a broadcast merge zeros, the identity), so no
// key is counted twice.  Each level is 8 DPP moves and 32 independent min/max: a few hundred
// cycles in all, against k dependent rounds of a wave-wide maximum.
template <int CTRL, int ROWS>
__device__ __forceinline__ void top8_merge(uint32_t (&a)[8]) {
  uint32_t b[8], c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a[i], CTRL, ROWS, 0xf, false);
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = max(a[i], b[7 - i]);
#pragma unroll
  for (int d = 4; d >= 1; d >>= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if ((i & d) == 0) {
        const uint32_t hi = max(c[i], c[i + d]), lo = min(c[i], c[i + d]);
        c[i] = hi;
        c[i + d] = lo;
      }
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = c[i];
}

// keys: this lane's PER keys (0 = empty), descending.  Returns the wave's 8 largest keys,
// descending, uniform.
template <int PER>
__device__ __forceinline__ void wave_top8(const uint32_t (&keys)[PER], uint32_t (&top)[8]) {
  uint32_t a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = i < PER ? keys[i] : 0u;
  top8_merge<0xb1, 0xf>(a);   // lane ^ 1
  top8_merge<0x4e, 0xf>(a);   // lane ^ 2
  top8_merge<0x124, 0xf>(a);  // row_ror:4
  top8_merge<0x128, 0xf>(a);  // row_ror:8: the row's 8 largest in every lane of the row
  top8_merge<0x142, 0xa>(a);  // row_bcast:15 into rows 1 and 3
  top8_merge<0x143, 0xc>(a);  // row_bcast:31 into rows 2 and 3: lane 63 holds the wave's
#pragma unroll
  for (int i = 0; i < 8; ++i) top[i] = (uint32_t)__builtin_amdgcn_readlane((int)a[i], 63);
}

// The top-k SET of one token (k <= 8) with no slot order and no scores: its expert ids in
// ascending id order in ids[0, k) (0xffffffff past k), uniform.  The keys and their order are
// route_token's, so the set is the same.
template <int PER>
__device__ __forceinline__ void route_set8(const uint16_t *__restrict__ l, int E, int k, uint32_t (&ids)[8]) {
  const int lane = (int)(threadIdx.x & 63);
  uint32_t pb[PER];
  route_probabilities<PER>(l, E, pb);
  uint32_t cand[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    cand[i] = e < E ? ((pb[i] << 16) | (uint32_t)e) + 1u : 0u;
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
  uint32_t top[8];
  wave_top8<PER>(cand, top);
#pragma unroll
  for (int i = 0; i < 8; ++i) ids[i] = i < k ? (top[i] - 1u) & 0xffffu : 0xffffffffu;
  // ascending ids: odd-even transposition over the 8 uniform values
#pragma unroll
  for (int pass = 0; pass < 8; ++pass)
#pragma unroll
    for (int i = pass & 1; i + 1 < 8; i += 2) {
      const uint32_t lo = min(ids[i], ids[i + 1]), hi = max(ids[i], ids[i + 1]);
      ids[i] = lo;
      ids[i + 1] = hi;
    }
}

// ------------------------------------------------------------------ MLX CPU argpartition order
//
// MLX's CPU argpartition (the oracle the reference's routing is checked against) fills an
// index vector 0..E-1 and runs std::nth_element(first, first + kth, last, comp) on it with
// comp(a, b) = v[a] < v[b] || (v[a] == v[b] && a < b); the slice [kth, E) is the top-k in the
// order that algorithm leaves.  On x86-64 Linux that is libstdc++'s introselect:
//   depth = 2 * floor(log2 n); while the range [f, l) holds more than 3 elements: after
//   `depth` partitions, a heap selection of [f, nth] over [f, l) and a swap of f and nth end
//   it; otherwise the median of a[f+1], a[mid], a[l-1] is swapped to f and the rest is
//   Hoare-partitioned around it (cut = first position not below the pivot), and the search
//   continues in [cut, l) if cut <= nth, else in [f, cut); a range of <= 3 is insertion-sorted.
// The device restates those steps on keys (bf16(p) << 16 | expert), which are unique and
// order exactly as comp orders the indices.  The Hoare partition runs wave-parallel: with Lc
// keys below the pivot in [f+1, l), cut = f + 1 + Lc, and the partition swaps the m-th key
// above the pivot in [f+1, cut) (counted from the left) with the m-th key below it in [cut, l)
// (counted from the right), for every m -- the pairs its two scanning pointers meet.  Ballots
// give each key its rank; two LDS tables pair the positions.

// Keeps this wave's later LDS accesses after its earlier ones in program order.  The LDS
// unit executes one wave's DS instructions in order, so a read issued after a write sees it
// (no wait needed); only the compiler must not move them.
__device__ __forceinline__ void wave_lds_order() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// libstdc++'s __adjust_heap followed by __push_heap on the max-heap b[0, len) (one lane).
__device__ __forceinline__ void heap_adjust(uint32_t *b, int hole, int len, uint32_t value) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (b[child] < b[child - 1]) child--;
    b[hole] = b[child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    b[hole] = b[child - 1];
    hole = child - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && b[parent] < value) {
    b[hole] = b[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  b[hole] = value;
}

// One median-of-three Hoare partition of [f, l) (C chunks of 64 positions cover [f + 1, l));
// returns cut.  Branch-free: lanes 0-3 fetch the three median candidates and a[f] in one
// read, every store is unconditional (lanes with nothing to store write their own word of
// `spare`, 64 words), so a step is two dependent LDS round trips and straight-line code.
template <int C>
__device__ __forceinline__ int hoare_step(uint32_t *a, uint32_t *pg, uint32_t *pl, uint32_t *spare, int f, int l) {
  const int lane = (int)(threadIdx.x & 63);
  // the median of a[f + 1], a[mid], a[l - 1] becomes the pivot at f (__move_median_to_first)
  const int mid = f + ((l - f) >> 1);
  const uint32_t cand = a[lane == 0 ? f + 1 : lane == 1 ? mid : lane == 2 ? l - 1 : f];
  uint32_t key[C];
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int p = f + 1 + lane + 64 * i;
    key[i] = a[p < l ? p : l - 1];
  }
  const uint32_t x = (uint32_t)__builtin_amdgcn_readlane((int)cand, 0);
  const uint32_t y = (uint32_t)__builtin_amdgcn_readlane((int)cand, 1);
  const uint32_t z = (uint32_t)__builtin_amdgcn_readlane((int)cand, 2);
  const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)cand, 3);
  int pos;
  uint32_t piv;
  if (x < y) {
    if (y < z) pos = mid, piv = y;
    else if (x < z) pos = l - 1, piv = z;
    else pos = f + 1, piv = x;
  } else if (x < z) pos = f + 1, piv = x;
  else if (y < z) pos = l - 1, piv = z;
  else pos = mid, piv = y;
  // ranks of the keys of [f + 1, l) above and below the pivot, counted from the left
  int gr[C], lr[C];
  bool gt[C], lt[C];
  int nl = 0, ng = 0;
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int p = f + 1 + lane + 64 * i;
    const bool valid = p < l;
    key[i] = p == pos ? o : key[i];  // the swap of the median to f
    gt[i] = valid && key[i] > piv;
    lt[i] = valid && key[i] < piv;
    const uint64_t bg = __ballot(gt[i]), bl = __ballot(lt[i]);
    gr[i] = ng + lanes_below(bg);
    lr[i] = nl + lanes_below(bl);
    ng += __popcll(bg);
    nl += __popcll(bl);
  }
  const int cut = f + 1 + nl;
  // the median swap (lane 0: a[f], lane 1: a[pos]), issued before the moves below
  *(lane == 0 ? a + f : lane == 1 ? a + pos : spare + lane) = lane == 0 ? piv : o;
  // pair tables: position of the m-th key above the pivot left of cut, of the m-th key below
  // it from the right at or after cut; then each moving key reads its partner's position
  bool left[C], right[C];
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int p = f + 1 + lane + 64 * i;
    left[i] = gt[i] && p < cut;
    right[i] = lt[i] && p >= cut;
    *(left[i] ? pg + gr[i] : right[i] ? pl + (nl - 1 - lr[i]) : spare + lane) = (uint32_t)p;
  }
  wave_lds_order();
  uint32_t dst[C];
#pragma unroll
  for (int i = 0; i < C; ++i) dst[i] = *(left[i] ? pl + gr[i] : right[i] ? pg + (nl - 1 - lr[i]) : spare + lane);
#pragma unroll
  for (int i = 0; i < C; ++i) *(left[i] || right[i] ? a + dst[i] : spare + lane) = key[i];
  wave_lds_order();
  return cut;
}

// std::nth_element(a, a + nth, a + n) over the unique keys a[0, n) in LDS, as libstdc++ runs
// it (see above).  One wave; n <= 64 * PER; pg and pl hold 32 * PER words each, spare 64.
// Each step partitions in as many 64-position chunks as its range needs.  The heap
// selection (reached only after 2 floor(log2 n) unbalanced partitions, i.e. adversarial keys)
// runs on one lane.
template <int PER>
__device__ __forceinline__ void nth_element_wave(uint32_t *a, uint32_t *pg, uint32_t *pl, uint32_t *spare, int n,
                                                 int nth) {
  const int lane = (int)(threadIdx.x & 63);
  if (n <= 0 || nth >= n) return;
  int f = 0, l = n, depth = 2 * (31 - __builtin_clz((unsigned)n));
  while (l - f > 3) {
    if (depth == 0) {
      if (lane == 0) {
        // __heap_select(f, nth + 1, l): make_heap over [f, nth], then every smaller key of
        // (nth, l) replaces the heap's top; then the swap of f and nth
        uint32_t *b = a + f;
        const int len = nth + 1 - f;
        if (len >= 2)
          for (int parent = (len - 2) / 2;; --parent) {
            heap_adjust(b, parent, len, b[parent]);
            if (parent == 0) break;
          }
        for (int i = nth + 1; i < l; ++i) {
          const uint32_t v = a[i];
          if (v < b[0]) {
            a[i] = b[0];
            heap_adjust(b, 0, len, v);
          }
        }
        const uint32_t t = a[f];
        a[f] = a[nth];
        a[nth] = t;
      }
      wave_lds_order();
      return;
    }
    --depth;
    // as many 64-position chunks as [f + 1, l) needs (a step's ballots and moves run per chunk)
    const int len = l - f;
    constexpr int C2 = PER < 2 ? PER : 2, C4 = PER < 4 ? PER : 4;
    const int cut = len <= 65 ? hoare_step<1>(a, pg, pl, spare, f, l)
                    : len <= 129 ? hoare_step<C2>(a, pg, pl, spare, f, l)
                    : len <= 257 ? hoare_step<C4>(a, pg, pl, spare, f, l)
                                 : hoare_step<PER>(a, pg, pl, spare, f, l);
    if (cut <= nth) f = cut;
    else l = cut;
  }
  if (lane == 0) {
    // __insertion_sort of at most 3 unique keys: ascending
    for (int i = f + 1; i < l; ++i) {
      const uint32_t v = a[i];
      int j = i;
      while (j > f && v < a[j - 1]) {
        a[j] = a[j - 1];
        --j;
      }
      a[j] = v;
    }
  }
  wave_lds_order();
}

// LDS words route_token_exact needs per routing wave: the keys (64 * PER), the partition's two
// pair tables (32 * PER each) and 64 spare words.
template <int PER>
constexpr int kSelectWords = 128 * PER + 64;

// One token's routing with MLX CPU argpartition's slice order (see above): lane j < k returns
// slot j's expert and (renormalised in slot order) score.  sel = kSelectWords<PER> words and
// sh = KMAX words (16-byte aligned) of this wave's LDS.
template <int PER, int KMAX>
__device__ __forceinline__ void route_token_exact(const uint16_t *__restrict__ l, int E, int k, int normalize,
                                                  uint32_t *sel, uint32_t *sh, uint32_t &out_idx,
                                                  uint32_t &out_score) {
  uint32_t *arr = sel;
  const int lane = (int)(threadIdx.x & 63);
  uint32_t pb[PER];
  route_probabilities<PER>(l, E, pb);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    if (e < E) arr[e] = (pb[i] << 16) | (uint32_t)e;
  }
  wave_lds_order();
  nth_element_wave<PER>(arr, sel + 64 * PER, sel + 96 * PER, sel + 128 * PER, E, E - k);
  const uint32_t key = arr[E - k + (lane < k ? lane : 0)];
  out_idx = key & 0xffffu;
  out_score = route_scores<KMAX>(key >> 16, k, normalize, sh);
}

}  // namespace astro
