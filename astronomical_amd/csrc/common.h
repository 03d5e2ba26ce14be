// Device helpers shared by the gfx950 kernels: bf16 bit conversions, the
// deterministic exp used by softmax/sigmoid, wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace astro {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// IEEE round-to-nearest-even fp32 -> bf16 on the bit pattern, NaN kept quiet with its sign and
// upper payload ((u >> 16) | 0x40): gfx950's v_cvt_pk_bf16_f32 (the compiler's float -> __bf16,
// with fp32 denormals kept) returns exactly these bits for all 2^32 inputs
// (astro_moe_selftest_bf16_rounding checks every one against the bit-pattern rounding).
__device__ __forceinline__ uint32_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
// the same rounding on the bit pattern (the definition the conversion is checked against)
__device__ __forceinline__ uint32_t f2bf_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) | 0x40u) : rounded;
}

// exp(x): Cody-Waite reduction x = n ln2 + r (|r| <= ln2/2), degree-7 Taylor polynomial
// with explicit fma, exact power-of-two scale; e^x below e^-80 is 0 so no subnormal is
// produced.  Only IEEE mul/fma/rint are used, so the host restatement of the same
// steps returns identical bits.  Branch-free: the argument is clamped to [-81, 89] for the
// arithmetic and the special cases (NaN, overflow, underflow) are selected at the end.
__device__ __forceinline__ float det_expf(float x) {
#pragma clang fp contract(off)
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -81.0f), 89.0f);
  const float n = __builtin_rintf(xc * 1.44269502162933349609375f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
  r = __builtin_fmaf(-n, 1.42860676533018704e-6f, r);
  float p = (float)(1.0 / 5040.0);
  p = __builtin_fmaf(p, r, (float)(1.0 / 720.0));
  p = __builtin_fmaf(p, r, (float)(1.0 / 120.0));
  p = __builtin_fmaf(p, r, (float)(1.0 / 24.0));
  p = __builtin_fmaf(p, r, (float)(1.0 / 6.0));
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  const bool big = ni > 127;  // 2^128 is not a float: scale by 2 * 2^127
  p = big ? p * 2.0f : p;
  ni = big ? ni - 1 : ni;
  float res = p * __uint_as_float((uint32_t)(ni + 127) << 23);
  res = x > 88.72283172607421875f ? __builtin_inff() : res;
  res = x < -80.0f ? 0.0f : res;
  return x != x ? x : res;
}

__device__ __forceinline__ float det_sigmoid(float v) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + det_expf(-v));
}

// bf16(det_sigmoid(g)) for every g, mostly without det_sigmoid's exp and IEEE division.
// 1 / (1 + 2^(-g log2 e)) on the hardware exp2 and reciprocal (1 ulp each), the exponent
// -g log2 e carried with its rounding error (log2 e as a two-float sum, the product's error by
// fma) and folded back as 2^x (1 + err ln 2): within 2 fp32 ulps of det_sigmoid over every bf16
// g with |g| <= 16.  An error that small changes the bf16 rounding only when the fp32 value is
// within a few ulps of a bf16 rounding midpoint (low 16 bits 0x8000): within 16 ulps of one,
// and for |g| > 16 or NaN, det_sigmoid decides.  Both paths round to the same bf16, so the
// result is det_sigmoid's for every input (the SwiGLU parity test sweeps all 2^16 bf16 gates).
__device__ __forceinline__ float sigmoid_bf(float g) {
#pragma clang fp contract(off)
  const float l2e_hi = 1.44269502162933349609375f, l2e_lo = 1.925963033500011079e-8f;
  const float x = -g * l2e_hi;
  const float xerr = __builtin_fmaf(-g, l2e_hi, -x) + -g * l2e_lo;
  const float e = __builtin_amdgcn_exp2f(x) * __builtin_fmaf(xerr, 0.693147180559945309f, 1.0f);
  float s = __builtin_amdgcn_rcpf(1.0f + e);
  const uint32_t near_mid = (__float_as_uint(s) & 0xffffu) - (0x8000u - 16u);
  if (!(__builtin_fabsf(g) <= 16.0f) || near_mid <= 32u) s = det_sigmoid(g);
  return round_bf(s);
}

// inputs (0, 4), (1, 5), (2, 6), (3, 7) of 8 consecutive bf16 values: the pairing of the
// exact-code GEMM's 4-bit unpack
__device__ __forceinline__ u32x4 pair_code_order(const u32x4 &d) {
  u32x4 a;
  a[0] = (d[0] & 0xffffu) | (d[2] << 16);
  a[1] = (d[0] >> 16) | (d[2] & 0xffff0000u);
  a[2] = (d[1] & 0xffffu) | (d[3] << 16);
  a[3] = (d[1] >> 16) | (d[3] & 0xffff0000u);
  return a;
}

// The fp32 sum of the g inputs at src (g / 8 pieces of 8 bf16), in input order: one group's
// sum for the exact-code GEMM's affine terms; with dst, also the inputs in the codes' pairing.
__device__ __forceinline__ float group_sum_paired(const u32x4 *src, int g, u32x4 *dst) {
  float sum = 0.0f;
  for (int c = 0; c < g / 8; ++c) {
    const u32x4 v = src[c];
#pragma unroll
    for (int w = 0; w < 4; ++w) sum = (sum + bf_lo(v[w])) + bf_hi(v[w]);
    if (dst) dst[c] = pair_code_order(v);
  }
  return sum;
}

// SwiGLU with the reference's three bf16 roundings (mlx_compiled_swiglu.rs:66-86):
// s = bf16(sigmoid(g)); a = bf16(g*s); out = bf16(a*u).
__device__ __forceinline__ uint32_t swiglu_bf(float g, float u) {
#pragma clang fp contract(off)
  const float s = sigmoid_bf(g);
  const float a = round_bf(g * s);
  return f2bf(a * u);
}

// One output element of the weighted combine (weighted_sum.rs:16-33 sorted / :112-119
// unsorted) followed by the shared expert's gated add (output_combination.rs:40-42):
// v[j] = expert row values of the token's k slots (slot order), s[j] = their scores.
template <bool SORTED, int KMAX>
__device__ __forceinline__ uint32_t combine_element(const float *v, const float *s, int k) {
#pragma clang fp contract(off)
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    const float nxt = SORTED ? __builtin_fmaf(v[j], s[j], acc) : acc + round_bf(v[j] * s[j]);
    acc = j < k ? nxt : acc;
  }
  return f2bf(acc);
}
__device__ __forceinline__ uint32_t shared_gated_add(uint32_t sparse_bits, float shared_value,
                                                     float gate_bf) {
#pragma clang fp contract(off)
  return f2bf(bf2f(sparse_bits) + round_bf(shared_value * gate_bf));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Canonical sum over the 64 lanes of a wave (the softmax denominator; the host oracle
// reproduces it bit for bit): the butterfly new[j] = v[j] + v[j ^ off] for
// off = 1, 2, 4, 8, 16, 32, value of lane 0.  Offsets 1 and 2 are DPP quad permutes; after
// them values are uniform within quads, so the half-row and row mirrors pair the same
// partial sums as offsets 4 and 8; the last two levels add the four row sums as
// (row0 + row1) + (row2 + row3).  Returns the sum in every lane.
__device__ __forceinline__ float wave_sum(float v) {
#pragma clang fp contract(off)
  v = v + dpp_f32<0xb1>(v);   // quad_perm [1,0,3,2]: lane j ^ 1
  v = v + dpp_f32<0x4e>(v);   // quad_perm [2,3,0,1]: lane j ^ 2
  v = v + dpp_f32<0x141>(v);  // row_half_mirror: the other quad of the 8-lane half
  v = v + dpp_f32<0x140>(v);  // row_mirror: the other half of the 16-lane row
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)v, off, kWave);
    v = o > v ? o : v;
  }
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// ---- RMS norm pieces shared by the standalone kernel and the decode router kernel
// r = bf16(h + a) of 8 elements (a null: r = h)
__device__ __forceinline__ u32x4 rms_residual(const u32x4 &h, const u32x4 *a) {
#pragma clang fp contract(off)
  if (!a) return h;
  const u32x4 av = *a;
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = f2bf(bf_lo(h[i]) + bf_lo(av[i])) | (f2bf(bf_hi(h[i]) + bf_hi(av[i])) << 16);
  return r;
}
// part + r_0^2 + ... + r_7^2, in element order
__device__ __forceinline__ float rms_partial(const u32x4 &r, float part) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = bf_lo(r[i]), hi = bf_hi(r[i]);
    part = part + lo * lo;
    part = part + hi * hi;
  }
  return part;
}
// the workgroup (256 threads) total: canonical butterfly per wave, then (w0 + w1) + (w2 + w3);
// wsum: 4 floats of LDS; every thread returns the total
__device__ __forceinline__ float rms_total(float part, float *wsum) {
#pragma clang fp contract(off)
  const float ws = wave_sum(part);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ws;
  __syncthreads();
  const float t = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
  __syncthreads();  // wsum may be reused
  return t;
}
__device__ __forceinline__ float rms_inverse(float total, int H, float eps) {
#pragma clang fp contract(off)
  return 1.0f / __builtin_sqrtf(total / (float)H + eps);
}
// n = bf16(w * bf16(r * inv)) of 8 elements
__device__ __forceinline__ u32x4 rms_apply(const u32x4 &r, const u32x4 &w, float inv) {
#pragma clang fp contract(off)
  u32x4 n;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    n[i] = f2bf(bf_lo(w[i]) * round_bf(bf_lo(r[i]) * inv)) | (f2bf(bf_hi(w[i]) * round_bf(bf_hi(r[i]) * inv)) << 16);
  return n;
}

// DPP rotation of a value within each 16-lane row (row_ror:n, n = 1..15).
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xf, 0xf, false));
}
template <int N>
__device__ __forceinline__ uint32_t row_ror_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + N, 0xf, 0xf, false);
}

// Sum over each 16-lane row; every lane of the row receives its row's sum.  For
// reductions whose summation order does not need to be reproduced elsewhere.
__device__ __forceinline__ float row_sum(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

// Sum over the wave (DPP within rows, then the four row sums); uniform result.
__device__ __forceinline__ float wave_sum_fast(float v) {
  v = row_sum(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// One affine row (BITS-bit codes, one bf16 scale and bias per group) times one bf16 input row
// of K (a multiple of 32) on one wave: lane l covers inputs 32l.. of each 2048-wide chunk,
// dequantising in fp32 (scale*q + bias) and accumulating x*w with fma; the wave sum in every
// lane.
template <int BITS>
__device__ __forceinline__ float qgemv_row_wave(const uint16_t *__restrict__ xr, int K, const uint32_t *__restrict__ wr,
                                                const uint16_t *__restrict__ sr, const uint16_t *__restrict__ br,
                                                int group) {
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  for (int k0 = lane * 32; k0 < K; k0 += 64 * 32) {
    const float s = bf2f(sr[k0 / group]), b = bf2f(br[k0 / group]);
    const u32x4 *xp = (const u32x4 *)(xr + k0);
    float xv[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 q = xp[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[8 * c + 2 * i] = bf_lo(q[i]);
        xv[8 * c + 2 * i + 1] = bf_hi(q[i]);
      }
    }
    const uint32_t *wp = wr + k0 * BITS / 32;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t word = wp[i * BITS / 32];
      const float q = (float)((word >> ((i * BITS) & 31)) & ((1u << BITS) - 1u));
      acc = __builtin_fmaf(xv[i], __builtin_fmaf(s, q, b), acc);
    }
  }
  return wave_sum_fast(acc);
}

// Maximum over the wave of unsigned keys with DPP only (quad permutes, row rotations, then
// row_bcast:15 / row_bcast:31 fold the rows into lane 63) and one readlane: a single
// vector-to-scalar transfer.  Uniform result.
__device__ __forceinline__ uint32_t wave_max_u32_bcast(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false));   // lane ^ 1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false));   // lane ^ 2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false));  // row_ror:4
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false));  // row_ror:8
  // rows 1 and 3 take lane 15 / 47 of the row below; rows 2 and 3 then take lane 31
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xa, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xc, 0xf, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ float wave_max_bcast(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xa, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Maximum over the wave of unsigned keys; uniform result.
__device__ __forceinline__ uint32_t wave_max_u32_fast(uint32_t v) {
  v = max(v, row_ror_u32<8>(v));
  v = max(v, row_ror_u32<4>(v));
  v = max(v, row_ror_u32<2>(v));
  v = max(v, row_ror_u32<1>(v));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(r0, r1), max(r2, r3));
}

__device__ __forceinline__ float wave_max_fast(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  v = fmaxf(v, row_ror<1>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

}  // namespace astro
