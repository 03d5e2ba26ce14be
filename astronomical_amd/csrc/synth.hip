// Seeded synthetic inputs on the device (benchmark and test harness; no counterpart in
// the reference).  Same counter-based streams as astronomical_amd/synthetic.py:
// element i of a tensor with stream key K draws splitmix64(K + i).
#include "common.h"
#include "../../include/astro_moe.h"

namespace astro {

namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ double unit53(uint64_t h) { return (double)(h >> 11) * 0x1.0p-53; }

__device__ __forceinline__ double normal_at(uint64_t key, int64_t i) {
  const uint64_t h1 = splitmix64(key + 2ull * (uint64_t)i);
  const uint64_t h2 = splitmix64(key + 2ull * (uint64_t)i + 1ull);
  const double u1 = ((double)(h1 >> 11) + 0.5) * 0x1.0p-53;
  const double u2 = unit53(h2);
  return sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2);
}

__device__ __forceinline__ uint16_t f64_to_bf16(double v) { return (uint16_t)f2bf((float)v); }

__global__ void words_kernel(uint32_t *out, int64_t n, uint64_t key) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = (uint32_t)splitmix64(key + (uint64_t)i);
}

__global__ void uniform_kernel(uint16_t *out, int64_t n, uint64_t key, double lo, double hi) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = f64_to_bf16(lo + unit53(splitmix64(key + (uint64_t)i)) * (hi - lo));
}

__global__ void biases_kernel(uint16_t *out, const uint16_t *scales, int64_t n, uint64_t key,
                              double center, double noise) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    double b = -center * (double)bf2f(scales[i]);
    if (noise != 0.0) b += noise * normal_at(key, i);
    out[i] = f64_to_bf16(b);
  }
}

__global__ void normal_kernel(uint16_t *out, int64_t n, uint64_t key, double scale) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = f64_to_bf16(scale * normal_at(key, i));
}

// one block per token: x / sqrt(mean(x^2) + 1e-6), float64, then bf16
__global__ __launch_bounds__(256) void activations_kernel(uint16_t *out, int hidden, uint64_t key) {
  __shared__ double part[256];
  const int t = blockIdx.x;
  double ss = 0.0;
  for (int h = threadIdx.x; h < hidden; h += 256) {
    const double v = normal_at(key, (int64_t)t * hidden + h);
    ss += v * v;
  }
  part[threadIdx.x] = ss;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) part[threadIdx.x] += part[threadIdx.x + off];
    __syncthreads();
  }
  const double denom = sqrt(part[0] / hidden + 1e-6);
  for (int h = threadIdx.x; h < hidden; h += 256)
    out[(int64_t)t * hidden + h] = f64_to_bf16(normal_at(key, (int64_t)t * hidden + h) / denom);
}

dim3 grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return dim3((unsigned)b);
}

}  // namespace
}  // namespace astro

using namespace astro;

extern "C" int astro_synth_words(uint32_t *out, int64_t n, uint64_t key, void *stream) {
  if (n <= 0) return ASTRO_MOE_OK;
  hipLaunchKernelGGL(words_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, out, n, key);
  return hipGetLastError() == hipSuccess ? ASTRO_MOE_OK : ASTRO_MOE_HIP_ERROR;
}

extern "C" int astro_synth_uniform_bf16(uint16_t *out, int64_t n, uint64_t key, double lo,
                                        double hi, void *stream) {
  if (n <= 0) return ASTRO_MOE_OK;
  hipLaunchKernelGGL(uniform_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, out, n, key,
                     lo, hi);
  return hipGetLastError() == hipSuccess ? ASTRO_MOE_OK : ASTRO_MOE_HIP_ERROR;
}

extern "C" int astro_synth_affine_biases(uint16_t *out, const uint16_t *scales, int64_t n,
                                         uint64_t key, double center, double noise,
                                         void *stream) {
  if (n <= 0) return ASTRO_MOE_OK;
  hipLaunchKernelGGL(biases_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, out, scales,
                     n, key, center, noise);
  return hipGetLastError() == hipSuccess ? ASTRO_MOE_OK : ASTRO_MOE_HIP_ERROR;
}

extern "C" int astro_synth_normal_bf16(uint16_t *out, int64_t n, uint64_t key, double scale,
                                       void *stream) {
  if (n <= 0) return ASTRO_MOE_OK;
  hipLaunchKernelGGL(normal_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, out, n, key,
                     scale);
  return hipGetLastError() == hipSuccess ? ASTRO_MOE_OK : ASTRO_MOE_HIP_ERROR;
}

extern "C" int astro_synth_activations(uint16_t *out, int32_t tokens, int32_t hidden,
                                       uint64_t key, void *stream) {
  if (tokens <= 0) return ASTRO_MOE_OK;
  hipLaunchKernelGGL(activations_kernel, dim3(tokens), dim3(256), 0, (hipStream_t)stream, out,
                     hidden, key);
  return hipGetLastError() == hipSuccess ? ASTRO_MOE_OK : ASTRO_MOE_HIP_ERROR;
}
