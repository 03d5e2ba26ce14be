// Decode path of the block (T <= 8 tokens, T*k <= 64 assignments): wavefront GEMVs
// instead of MFMA tiles, three kernels per layer:
//   D1  router GEMV (one wave per expert row);
//   D2  the shared expert's gate/up + SwiGLU and its output gate (no routing needed), and
//       routing (softmax/top-k, the sort of the assignments, the distinct-expert table),
//       recomputed by every routed workgroup, then the routed gate/up GEMV + SwiGLU: one
//       wave per (gate row, up row) pair of one selected expert, every token routed to it;
//   D3  per token: down GEMV rows of its k experts and of the shared expert (16 lanes per
//       row, the participants spread over 4 waves), then the weighted combine and the
//       shared expert's gated add.
// Affine rows are read once per distinct expert with 16 B per lane loads.  4-bit codes are
// turned into bf16 pairs (128 + q) with one and/or per pair and multiplied by
// v_dot2_f32_bf16; the per-group affine terms are applied per 32-input chunk:
//   sum_j x_j (s q_j + b) = s * sum_j (128 + q_j) x_j + (b - 128 s) * sum_j x_j.
#include "decode_dev.h"

namespace astro {

bool decode_supported(const DecodeArgs &a) {
  const bool router_ok = a.router_w ? !a.rq_w
                                    : a.rq_w && (a.rq_bits == 4 || a.rq_bits == 8) && a.rq_group >= 32;
  return a.T >= 1 && a.T <= 8 && a.A <= 64 && router_ok && a.H % 32 == 0 &&
         a.H <= 4096 && a.I % 32 == 0 && a.I <= 1024 && a.Is % 32 == 0 && a.Is <= 1024 &&
         a.E <= 1024 && a.k >= 1 && a.k <= kDecodeMaxK && (a.gu_bits == 4 || a.gu_bits == 8) &&
         (a.dn_bits == 4 || a.dn_bits == 8) && a.gu_group >= 32 && a.dn_group >= 32 &&
         (a.Is == 0 || (a.sd_bits == a.dn_bits && (a.sg_bits == 4 || a.sg_bits == 8) &&
                        (a.sz_bits == 4 || a.sz_bits == 8) && a.sd_group >= 32 &&
                        a.sg_group >= 32 && a.sz_group >= 32)) &&
         (!a.norm_w || ((size_t)a.T * a.H * 2 <= (size_t)kDecodeStepLds && a.H % 8 == 0 && a.h_in &&
                        a.r_out && a.x_out && a.x == a.x_out && a.ffn_out));
}

hipError_t launch_decode_block(const DecodeArgs &a, hipStream_t s, const hipEvent_t *kev) {
  const int mt = a.T <= 1 ? 1 : a.T <= 2 ? 2 : a.T <= 4 ? 4 : 8;
  const hipEvent_t *e1 = kev ? kev : nullptr, *e2 = kev ? kev + 2 : nullptr,
                   *e3 = kev ? kev + 4 : nullptr;
  // D1: router rows (4 experts per block)
  if (mt == 1) launch_router<1>(a, a.router_blocks, s, e1);
  else if (mt == 2) launch_router<2>(a, a.router_blocks, s, e1);
  else if (mt == 4) launch_router<4>(a, a.router_blocks, s, e1);
  else launch_router<8>(a, a.router_blocks, s, e1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // routing once for a batch of tokens (kev[6..7], when given, time it)
  if (a.T >= kDecodeRouteOnceT) {
    const hipEvent_t *er = kev ? kev + 6 : nullptr;
    if (mt == 2) launch_route_mt<2>(a, s, er);
    else if (mt == 4) launch_route_mt<4>(a, s, er);
    else launch_route_mt<8>(a, s, er);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  // D2: shared gate/up, routing (T = 1), routed gate/up
  if (a.gu_bits == 8) {
    if (mt == 1) launch_decode_gate_up<8, 1>(a, s, e2);
    else if (mt == 2) launch_decode_gate_up<8, 2>(a, s, e2);
    else if (mt == 4) launch_decode_gate_up<8, 4>(a, s, e2);
    else launch_decode_gate_up<8, 8>(a, s, e2);
  } else {
    if (mt == 1) launch_decode_gate_up<4, 1>(a, s, e2);
    else if (mt == 2) launch_decode_gate_up<4, 2>(a, s, e2);
    else if (mt == 4) launch_decode_gate_up<4, 4>(a, s, e2);
    else launch_decode_gate_up<4, 8>(a, s, e2);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // D3: down projections and the combine
  if (a.dn_bits == 8) launch_down<8>(a, s, e3);
  else launch_down<4>(a, s, e3);
  return hipGetLastError();
}

}  // namespace astro
