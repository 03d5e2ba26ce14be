// Router softmax / top-k / renormalisation (routing.rs:16-48) and the stable
// sort-by-expert permutation (assignment_sort.rs:79-91) with the grouped-GEMM tile table.
#include "common.h"
#include "kernels.h"
#include "route_dev.h"

namespace astro {

namespace {

// One wave per token (route_token_exact in route_dev.h: the slice in the order MLX's CPU
// argpartition leaves it), four tokens per workgroup.  With ex.x set, waves 4..7 of the
// workgroup (launched with 8) do the same tokens' share of the work RouteExtras lists, beside
// the routing: their group sums and paired copies (group_sums_kernel's work, one lane per group,
// the same order of additions) and their shared-expert gates (qgemv_row_wave, as
// qgemv_rows_kernel), which then need no launches of their own.
template <int PER, int KMAX>
__global__ __launch_bounds__(512) void route_topk_kernel(const uint16_t *__restrict__ logits,
                                                         int T, int E, int k, int normalize,
                                                         uint32_t *__restrict__ idx,
                                                         uint16_t *__restrict__ scores, const RouteExtras ex) {
  __shared__ __attribute__((aligned(16))) uint32_t sh[4][KMAX];
  __shared__ uint32_t sel[4][kSelectWords<PER>];  // per wave: keys, the partition's pair tables
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int t = blockIdx.x * 4 + (wave & 3);
  if (t >= T) return;
  if (wave < 4) {
    uint32_t my_idx, my_score;
    route_token_exact<PER, KMAX>(logits + (int64_t)t * E, E, k, normalize, sel[wave], sh[wave], my_idx, my_score);
    if (lane < k) {
      idx[(int64_t)t * k + lane] = my_idx;
      scores[(int64_t)t * k + lane] = (uint16_t)my_score;
    }
    return;
  }
  if (ex.x && ex.z) {
    const uint16_t *xr = ex.x + (int64_t)t * ex.H;
    const float acc = ex.zbits == 8 ? qgemv_row_wave<8>(xr, ex.H, ex.zw, ex.zs, ex.zb, ex.zgroup)
                                    : qgemv_row_wave<4>(xr, ex.H, ex.zw, ex.zs, ex.zb, ex.zgroup);
    if (lane == 0) ex.z[t] = (uint16_t)f2bf(acc);
  }
  if (ex.x && ex.xsum) {
    const int G = ex.H / ex.g;
    for (int gi = lane; gi < G; gi += 64) {
      const u32x4 *src = (const u32x4 *)(ex.x + (int64_t)t * ex.H + (int64_t)gi * ex.g);
      u32x4 *dst = (u32x4 *)(ex.paired + (int64_t)t * ex.H + (int64_t)gi * ex.g);
      ex.xsum[(int64_t)t * G + gi] = group_sum_paired(src, ex.g, dst);
    }
  }
}

constexpr int kChunk = 1024;  // assignments per rank / place workgroup (16 waves)
constexpr int kMaxBuckets = 1025;  // experts <= 1024, plus the bucket of ids >= E

// Lanes of this wave whose bucket equals this lane's (invalid lanes match nothing): one
// ballot per bit of the bucket number.
__device__ __forceinline__ uint64_t same_bucket_lanes(uint32_t b, bool valid, int nbits) {
  uint64_t m = __ballot(valid);
  for (int i = 0; i < nbits; ++i) {
    const bool bit = (b >> i) & 1u;
    const uint64_t bal = __ballot(valid && bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

// Stable counting sort in two launches.
// rank: each workgroup takes kChunk consecutive assignments; every wave ranks its 64 ids
// (number of earlier lanes with the same bucket) and records, per bucket, its count; the
// workgroup then turns those into chunk-local ranks (earlier waves' counts + the in-wave
// rank) and writes the chunk's bucket histogram.
__global__ __launch_bounds__(kChunk) void sort_rank_kernel(const uint32_t *__restrict__ ids, int A,
                                                           int E, int nbits, uint32_t *__restrict__ hist,
                                                           uint32_t *__restrict__ local_rank) {
  extern __shared__ uint16_t wcnt[];  // [16 waves][E + 1] (a wave counts at most 64)
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int nb = E + 1;
  for (int i = threadIdx.x; i < 16 * nb; i += kChunk) wcnt[i] = 0;
  const int a = blockIdx.x * kChunk + threadIdx.x;
  const bool valid = a < A;
  const uint32_t id = valid ? ids[a] : 0u;
  const uint32_t b = id < (uint32_t)E ? id : (uint32_t)E;
  const uint64_t m = same_bucket_lanes(b, valid, nbits);
  const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
  const bool closes = (m >> lane) == 1ull;  // no later lane shares the bucket
  __syncthreads();
  if (valid && closes) wcnt[w * nb + b] = (uint16_t)(before + 1);
  __syncthreads();
  if (valid) {
    uint32_t r = before;
    for (int v = 0; v < w; ++v) r += wcnt[v * nb + b];
    local_rank[a] = r;
  }
  for (int e = threadIdx.x; e < nb; e += kChunk) {
    uint32_t c = 0;
#pragma unroll
    for (int v = 0; v < 16; ++v) c += wcnt[v * nb + e];
    hist[(size_t)blockIdx.x * nb + e] = c;
  }
}

// place: workgroup c (one per chunk, at least one) sums every chunk's histogram per bucket
// (total) and the histograms of chunks before c (pre), scans the totals into the bucket
// offsets, and scatters its chunk to offsets[bucket] + pre[bucket] + local rank.  Workgroup 0
// also writes offsets (E + 2 entries) and the tile table (tiles of kGemmBM rows, experts
// ascending).
__global__ __launch_bounds__(kChunk) void sort_place_kernel(
    const uint32_t *__restrict__ ids, int A, int E, const uint32_t *__restrict__ hist, int nchunks,
    const uint32_t *__restrict__ local_rank, uint32_t *__restrict__ sorted_order,
    uint32_t *__restrict__ inverse_order, uint32_t *__restrict__ sorted_ids,
    uint32_t *__restrict__ offsets, uint32_t *__restrict__ tile_expert,
    uint32_t *__restrict__ tile_row0, uint32_t *__restrict__ tile_count, uint32_t *__restrict__ xtiles) {
  __shared__ uint32_t base[kMaxBuckets];
  __shared__ uint32_t wsum[4][kChunk / 64];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int nb = E + 1;
  const int c = blockIdx.x;
  const int a = c * kChunk + threadIdx.x;
  const bool valid = a < A;
  const uint32_t id = valid ? ids[a] : 0u;
  const uint32_t lr = valid ? local_rank[a] : 0u;
  // thread e owns bucket e (E + 1 <= 1025 buckets: thread 0 also takes bucket 1024)
  auto sums = [&](int e, uint32_t &total, uint32_t &pre) {
    total = 0;
    pre = 0;
    if (e >= nb) return;
    for (int c0 = 0; c0 < nchunks; c0 += 16) {
      uint32_t h[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) h[u] = c0 + u < nchunks ? hist[(size_t)(c0 + u) * nb + e] : 0u;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        total += h[u];
        pre += c0 + u < c ? h[u] : 0u;
      }
    }
  };
  const int e = threadIdx.x;
  uint32_t total, pre;
  sums(e, total, pre);
  const uint32_t tiles = e < E ? (total + kGemmBM - 1) / kGemmBM : 0u;
  // tiles of more than kGemmBM / 2 rows (every full tile, and a last tile that large) come
  // first in the table and the smaller last tiles after all of them: the GEMMs deal tiles in
  // table order, so the light tiles fill the grid's last, partial round
  const uint32_t big = e < E ? total / kGemmBM + (total % kGemmBM > kGemmBM / 2 ? 1u : 0u) : 0u;
  // the exact-code GEMM's tiles: ceil(total / kXqRows) of balanced sizes per expert
  const uint32_t xt = e < E ? (total + kXqRows - 1) / kXqRows : 0u;
  uint32_t extra_total = 0, extra_pre = 0;
  if (threadIdx.x == 0 && nb > kChunk) sums(kChunk, extra_total, extra_pre);
  // block inclusive scans of total, tiles, big tiles and exact-code tiles
  uint32_t it = total, ip = tiles, ib = big, ix = xt;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)it, off, kWave);
    const uint32_t q = (uint32_t)__shfl_up((int)ip, off, kWave);
    const uint32_t g = (uint32_t)__shfl_up((int)ib, off, kWave);
    const uint32_t h = (uint32_t)__shfl_up((int)ix, off, kWave);
    if (lane >= off) {
      it += o;
      ip += q;
      ib += g;
      ix += h;
    }
  }
  if (lane == 63) {
    wsum[0][w] = it;
    wsum[1][w] = ip;
    wsum[2][w] = ib;
    wsum[3][w] = ix;
  }
  __syncthreads();
  uint32_t bt = 0, bp = 0, bb = 0, bx = 0, big_all = 0;
  for (int v = 0; v < w; ++v) {
    bt += wsum[0][v];
    bp += wsum[1][v];
    bb += wsum[2][v];
    bx += wsum[3][v];
  }
  for (int v = 0; v < kChunk / 64; ++v) big_all += wsum[2][v];
  const uint32_t off_e = bt + it - total;
  const uint32_t big0 = bb + ib - big;                      // big tiles of the buckets before e
  const uint32_t small0 = big_all + (bp + ip - tiles) - big0;  // after every big tile
  if (e < nb) {
    base[e] = off_e + pre;
    if (c == 0) {
      offsets[e] = off_e;
      for (uint32_t i = 0; i < tiles; ++i) {
        const uint32_t t = i < big ? big0 + i : small0;  // at most one small tile per bucket
        tile_expert[t] = (uint32_t)e;
        tile_row0[t] = off_e + i * kGemmBM;
      }
      if (xtiles) {
        // entries (expert | rows << 16, first row) from word 2 on; word 0 holds the count
        const uint32_t x0 = bx + ix - xt;
        for (uint32_t i = 0; i < xt; ++i) {
          const uint32_t r0 = (uint32_t)(((uint64_t)i * total) / xt);
          const uint32_t r1 = (uint32_t)(((uint64_t)(i + 1) * total) / xt);
          xtiles[2 + 2 * (x0 + i)] = (uint32_t)e | ((r1 - r0) << 16);
          xtiles[3 + 2 * (x0 + i)] = off_e + r0;
        }
      }
      if (e == nb - 1) {  // the last bucket's thread knows the totals
        offsets[nb] = (uint32_t)A;
        *tile_count = bp + ip;
        if (xtiles) xtiles[0] = bx + ix;
      }
    }
  }
  if (threadIdx.x == 0 && nb > kChunk) {
    // bucket 1024 (ids >= E when E = 1024): after every other bucket
    const uint32_t off_x = (uint32_t)A - extra_total;
    base[kChunk] = off_x + extra_pre;
    if (c == 0) {
      uint32_t nt = 0;  // tiles of buckets 0 .. 1023
      for (int v = 0; v < kChunk / 64; ++v) nt += wsum[1][v];
      offsets[kChunk] = off_x;
      offsets[nb] = (uint32_t)A;
      *tile_count = nt;
      if (xtiles) {
        uint32_t nx = 0;  // exact-code tiles of buckets 0 .. 1023
        for (int v = 0; v < kChunk / 64; ++v) nx += wsum[3][v];
        xtiles[0] = nx;
      }
    }
  }
  __syncthreads();
  if (valid) {
    const uint32_t b = id < (uint32_t)E ? id : (uint32_t)E;
    const uint32_t pos = base[b] + lr;
    sorted_order[pos] = (uint32_t)a;
    sorted_ids[pos] = id;
    inverse_order[a] = pos;
  }
}

}  // namespace

template <int KMAX>
void launch_route_k(const uint16_t *logits, int T, int E, int k, int normalize, uint32_t *idx,
                    uint16_t *scores, hipStream_t s, const RouteExtras &ex) {
  const dim3 grid((T + 3) / 4), block(ex.x ? 512 : 256);  // waves 4..7: the extras
  const int per = (E + 63) / 64;
  if (per <= 1)
    hipLaunchKernelGGL((route_topk_kernel<1, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores, ex);
  else if (per <= 2)
    hipLaunchKernelGGL((route_topk_kernel<2, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores, ex);
  else if (per <= 4)
    hipLaunchKernelGGL((route_topk_kernel<4, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores, ex);
  else if (per <= 8)
    hipLaunchKernelGGL((route_topk_kernel<8, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores, ex);
  else
    hipLaunchKernelGGL((route_topk_kernel<16, KMAX>), grid, block, 0, s, logits, T, E, k, normalize, idx, scores, ex);
}

hipError_t launch_route_topk(const uint16_t *logits, int T, int E, int k, int normalize,
                             uint32_t *idx, uint16_t *scores, hipStream_t s, const RouteExtras &ex) {
  if (T <= 0) return hipSuccess;
  if (ex.x && ex.xsum && (ex.g <= 0 || ex.g % 8 || ex.H % ex.g || !ex.paired)) return hipErrorInvalidValue;
  if (ex.x && ex.z && (ex.H % 32 || (ex.zbits != 4 && ex.zbits != 8) || ex.zgroup <= 0 || ex.zgroup % 32 || !ex.zw))
    return hipErrorInvalidValue;
  // KMAX bounds the renormalisation's unrolled slice sum
  if (k <= 8) launch_route_k<8>(logits, T, E, k, normalize, idx, scores, s, ex);
  else if (k <= 16) launch_route_k<16>(logits, T, E, k, normalize, idx, scores, s, ex);
  else launch_route_k<64>(logits, T, E, k, normalize, idx, scores, s, ex);
  return hipGetLastError();
}

int sort_max_tiles(int A, int E) { return A / kGemmBM + E + 1; }

int sort_max_xtiles(int A, int E) { return A / kXqRows + E + 1; }

size_t sort_scratch_bytes(int A, int E) {
  const size_t nchunks = ((size_t)A + kChunk - 1) / kChunk;
  return ((nchunks * ((size_t)E + 1) * 4 + 255) & ~(size_t)255) + (size_t)A * 4;
}

hipError_t launch_sort(const uint32_t *ids, int A, int E, uint32_t *sorted_order,
                       uint32_t *inverse_order, uint32_t *sorted_ids, uint32_t *offsets,
                       uint32_t *tile_expert, uint32_t *tile_row0, uint32_t *tile_count,
                       uint32_t *scratch, hipStream_t s, uint32_t *xtiles) {
  if (E < 1 || E + 1 > kMaxBuckets) return hipErrorInvalidValue;
  const int nchunks = (A + kChunk - 1) / kChunk;
  uint32_t *hist = scratch;
  uint32_t *local_rank = (uint32_t *)((char *)scratch + (((size_t)nchunks * (E + 1) * 4 + 255) & ~(size_t)255));
  const int nbits = 32 - __builtin_clz((unsigned)E);  // bits of the largest bucket number, E
  if (nchunks > 0) {
    hipLaunchKernelGGL(sort_rank_kernel, dim3(nchunks), dim3(kChunk), sizeof(uint16_t) * 16 * ((size_t)E + 1),
                       s, ids, A, E, nbits, hist, local_rank);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(sort_place_kernel, dim3(nchunks > 0 ? nchunks : 1), dim3(kChunk), 0, s, ids, A, E, hist,
                     nchunks, local_rank, sorted_order, inverse_order, sorted_ids, offsets, tile_expert,
                     tile_row0, tile_count, xtiles);
  return hipGetLastError();
}

}  // namespace astro
