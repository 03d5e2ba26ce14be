// Device helpers shared by the grouped GEMMs (gemm.hip, gemm_xq.hip): the tile of a
// workgroup, the barrier of the LDS rings and explicit vmcnt waits.
#pragma once

#include "common.h"
#include "kernels.h"

namespace astro {
namespace {

constexpr int BM = kGemmBM;  // rows per tile

// Workgroup -> (row tile, column tile).  Workgroups are dealt to the 8 XCDs round-robin by
// linear id (x fastest); the grid has a multiple of 8 row tiles.  Each XCD takes the row
// tiles x = xcd (mod 8), and its column tiles of one row tile come one after the other in
// its dispatch order, so they run together and share the activation tile in that XCD's L2.
__device__ __forceinline__ void tile_of_block(int &bx, int &by) {
  const int mt = (int)gridDim.x, nb = (int)gridDim.y;
  const int l = (int)blockIdx.x + (int)blockIdx.y * mt;
  const int xcd = l & 7, s = l >> 3;
  bx = (s / nb) * 8 + xcd;
  by = s - (s / nb) * nb;
}

// Tile of the launch: blocks x < split belong to problem a, the rest to problem b (a
// second GEMM fused into the same launch, e.g. the shared expert next to the routed
// experts).  A problem with a tile table is grouped: x indexes its tiles; otherwise row
// tiles are consecutive.  Returns false when the block has no work.  The problem is
// selected by value: taking the address of a kernel argument would copy both to scratch.
__device__ __forceinline__ bool gemm_tile(const GemmArgs &p, int bx, int by, bool second, int split, int nblocks,
                                          int &expert, int &row0, int &m_valid) {
  if (by >= nblocks) return false;
  const int x = second ? bx - split : bx;
  expert = 0;
  if (p.tile_expert) {
    if (x >= (int)*p.tile_count) return false;
    expert = (int)p.tile_expert[x];
    row0 = (int)p.tile_row0[x];
    m_valid = min(BM, (int)p.expert_offsets[expert + 1] - row0);
  } else {
    row0 = x * BM;
    m_valid = min(BM, p.M - row0);
  }
  return m_valid > 0;
}

// Workgroup barrier without the memory fence of __syncthreads (whose release would wait for
// every outstanding global->LDS load).  Each wave first waits for its own LDS accesses
// (lgkmcnt 0), so its LDS stores are visible and its LDS reads are done when it reaches the
// barrier; the async loads are covered by wait_vmcnt_le before it.  The asm statements
// also stop the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) with expcnt and lgkmcnt at their maxima (no wait on them); n is a
// compile-time constant at every call, so the switch folds to one instruction.  The empty asm
// keeps every memory access issued before the call ahead of the wait (the count relies on it).
__device__ __forceinline__ void wait_vmcnt_le(int n) {
  asm volatile("" ::: "memory");
  switch (n) {
#define ASTRO_WAITVM(N) \
  case N:               \
    __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | 0x0f70); \
    break;
#define ASTRO_WAITVM8(B) ASTRO_WAITVM(B) ASTRO_WAITVM(B + 1) ASTRO_WAITVM(B + 2) ASTRO_WAITVM(B + 3) \
  ASTRO_WAITVM(B + 4) ASTRO_WAITVM(B + 5) ASTRO_WAITVM(B + 6) ASTRO_WAITVM(B + 7)
    ASTRO_WAITVM8(0) ASTRO_WAITVM8(8) ASTRO_WAITVM8(16) ASTRO_WAITVM8(24)
    ASTRO_WAITVM8(32) ASTRO_WAITVM8(40) ASTRO_WAITVM8(48) ASTRO_WAITVM8(56)
#undef ASTRO_WAITVM8
#undef ASTRO_WAITVM
    default:
      __builtin_amdgcn_s_waitcnt(0x0f70);
      break;
  }
}

}  // namespace
}  // namespace astro
