// The decode path's gate/up kernels (D2) of one code width and token count, compiled once
// per (ASTRO_GU_BITS, ASTRO_GU_MT) pair so the many instantiations build in parallel.
#include "decode_dev.h"

#ifndef ASTRO_GU_BITS
#error "build with -DASTRO_GU_BITS=4|8 -DASTRO_GU_MT=1|2|4|8"
#endif

namespace astro {

template <int BITS, int MT>
void launch_decode_gate_up(const DecodeArgs &a, hipStream_t s, const hipEvent_t *ev) {
  launch_gate_up_mt<BITS, MT>(a, s, ev);
}

template void launch_decode_gate_up<ASTRO_GU_BITS, ASTRO_GU_MT>(const DecodeArgs &, hipStream_t, const hipEvent_t *);

}  // namespace astro
