// Router softmax / top-k / renormalisation (routing.rs:16-48) and the stable
// sort-by-expert permutation (assignment_sort.rs:79-91) with the grouped-GEMM tile table.
#include "common.h"
#include "kernels.h"
#include "route_dev.h"

namespace astro {

namespace {

// One wave per token (route_token in route_dev.h).
template <int PER, int KMAX>
__global__ __launch_bounds__(256) void route_topk_kernel(const uint16_t *__restrict__ logits,
                                                         int T, int E, int k, int normalize,
                                                         uint32_t *__restrict__ idx,
                                                         uint16_t *__restrict__ scores) {
  __shared__ __attribute__((aligned(16))) uint32_t sh[4][KMAX];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  uint32_t my_idx, my_score;
  route_token<PER, KMAX>(logits + (int64_t)t * E, E, k, normalize, sh[wave], my_idx, my_score);
  if (lane < k) {
    idx[(int64_t)t * k + lane] = my_idx;
    scores[(int64_t)t * k + lane] = (uint16_t)my_score;
  }
}

constexpr int kSortThreads = 1024;

// Histogram of expert ids (ids >= E counted in bucket E), exclusive scan -> offsets
// [E+2], and the tile table: tiles of kGemmBM rows, experts in ascending order.
__global__ __launch_bounds__(kSortThreads) void sort_count_kernel(
    const uint32_t *__restrict__ ids, int A, int E, uint32_t *__restrict__ offsets,
    uint32_t *__restrict__ tile_expert, uint32_t *__restrict__ tile_row0,
    uint32_t *__restrict__ tile_count) {
  extern __shared__ uint32_t sh[];
  uint32_t *cnt = sh;              // E + 1
  uint32_t *tbase = sh + E + 1;    // E + 1
  uint32_t *offs = sh + 2 * (E + 1); // E + 1
  for (int e = threadIdx.x; e <= E; e += kSortThreads) cnt[e] = 0;
  __syncthreads();
  for (int a = threadIdx.x; a < A; a += kSortThreads) {
    const uint32_t id = ids[a];
    atomicAdd(&cnt[id < (uint32_t)E ? id : (uint32_t)E], 1u);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0, tiles = 0;
    for (int e = 0; e <= E; ++e) {
      const uint32_t c = cnt[e];
      offsets[e] = run;
      offs[e] = run;
      tbase[e] = tiles;
      run += c;
      if (e < E) tiles += (c + kGemmBM - 1) / kGemmBM;
    }
    offsets[E + 1] = run;
    *tile_count = tiles;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSortThreads) {
    const uint32_t c = cnt[e], nt = (c + kGemmBM - 1) / kGemmBM;
    const uint32_t first = offs[e];
    for (uint32_t i = 0; i < nt; ++i) {
      tile_expert[tbase[e] + i] = (uint32_t)e;
      tile_row0[tbase[e] + i] = first + i * kGemmBM;
    }
  }
}

// One workgroup per bucket (expert, or the trailing out-of-range bucket).  Thread j
// owns a contiguous segment of slots; a block-wide exclusive scan of the per-segment
// match counts gives each match its rank, so ties keep ascending slot order (stable).
constexpr int kScatterThreads = 256;
__global__ __launch_bounds__(kScatterThreads) void sort_scatter_kernel(
    const uint32_t *__restrict__ ids, int A, int E, const uint32_t *__restrict__ offsets,
    uint32_t *__restrict__ sorted_order, uint32_t *__restrict__ inverse_order,
    uint32_t *__restrict__ sorted_ids) {
  __shared__ uint32_t wsum[kScatterThreads / 64];
  const uint32_t bucket = blockIdx.x;
  const uint32_t begin = offsets[bucket], count = offsets[bucket + 1] - begin;
  if (count == 0) return;
  const int seg = (A + kScatterThreads - 1) / kScatterThreads;
  const int a0 = threadIdx.x * seg, a1 = min(A, a0 + seg);
  auto bucket_of = [&](uint32_t id) { return id < (uint32_t)E ? id : (uint32_t)E; };
  // count pass: 16 independent loads in flight per step
  uint32_t mine = 0;
  for (int base = a0; base < a1; base += 16) {
    uint32_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = base + j < a1 ? ids[base + j] : 0u;
#pragma unroll
    for (int j = 0; j < 16; ++j) mine += (base + j < a1) && bucket_of(v[j]) == bucket;
  }
  // block exclusive scan of `mine`
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  uint32_t incl = mine;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)incl, off, kWave);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  uint32_t before = 0;
  for (int i = 0; i < w; ++i) before += wsum[i];
  uint32_t pos = begin + before + incl - mine;
  for (int base = a0; base < a1 && mine; base += 16) {
    uint32_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = base + j < a1 ? ids[base + j] : 0u;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int a = base + j;
      if (a < a1 && bucket_of(v[j]) == bucket) {
        sorted_order[pos] = (uint32_t)a;
        sorted_ids[pos] = v[j];
        inverse_order[a] = pos;
        ++pos;
        --mine;
      }
    }
  }
}

}  // namespace

template <int KMAX>
void launch_route_k(const uint16_t *logits, int T, int E, int k, int normalize, uint32_t *idx,
                    uint16_t *scores, hipStream_t s) {
  const dim3 grid((T + 3) / 4), block(256);
  const int per = (E + 63) / 64;
  if (per <= 1)
    hipLaunchKernelGGL((route_topk_kernel<1, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores);
  else if (per <= 2)
    hipLaunchKernelGGL((route_topk_kernel<2, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores);
  else if (per <= 4)
    hipLaunchKernelGGL((route_topk_kernel<4, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores);
  else if (per <= 8)
    hipLaunchKernelGGL((route_topk_kernel<8, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores);
  else
    hipLaunchKernelGGL((route_topk_kernel<16, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores);
}

hipError_t launch_route_topk(const uint16_t *logits, int T, int E, int k, int normalize,
                             uint32_t *idx, uint16_t *scores, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  // KMAX bounds the renormalisation's unrolled slice sum
  if (k <= 8) launch_route_k<8>(logits, T, E, k, normalize, idx, scores, s);
  else if (k <= 16) launch_route_k<16>(logits, T, E, k, normalize, idx, scores, s);
  else launch_route_k<64>(logits, T, E, k, normalize, idx, scores, s);
  return hipGetLastError();
}

int sort_max_tiles(int A, int E) { return A / kGemmBM + E + 1; }

hipError_t launch_sort(const uint32_t *ids, int A, int E, uint32_t *sorted_order,
                       uint32_t *inverse_order, uint32_t *sorted_ids, uint32_t *offsets,
                       uint32_t *tile_expert, uint32_t *tile_row0, uint32_t *tile_count,
                       hipStream_t s) {
  const size_t sh = sizeof(uint32_t) * 3 * ((size_t)E + 1);
  hipLaunchKernelGGL(sort_count_kernel, dim3(1), dim3(kSortThreads), sh, s, ids, A, E, offsets,
                     tile_expert, tile_row0, tile_count);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || A == 0) return err;
  hipLaunchKernelGGL(sort_scatter_kernel, dim3(E + 1), dim3(kScatterThreads), 0, s, ids, A, E,
                     offsets, sorted_order, inverse_order, sorted_ids);
  return hipGetLastError();
}

}  // namespace astro
