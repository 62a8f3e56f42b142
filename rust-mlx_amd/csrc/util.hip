// Synthetic-data generators and a math probe kernel.
#include "common.hpp"
#include "kernels.hpp"

namespace mx {

namespace {

__global__ void fill_bf16_kernel(uint16_t* __restrict__ dst, size_t count, uint64_t seed, int dist,
                                 float a, float b) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += size_t(gridDim.x) * blockDim.x) {
    const float v = dist == 0 ? rng_uniform(seed, i, a, b) : fmaf_(rng_normal(seed, i), a, b);
    dst[i] = f32_to_bf16(v);
  }
}

// One thread per 32-bit word of the packed code matrix.
__global__ void fill_codes_kernel(uint32_t* __restrict__ dst, int64_t rows, int k, int bits,
                                  uint64_t seed) {
  const int64_t words_per_row = (int64_t(k) * bits) >> 5;
  const int64_t total = rows * words_per_row;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t row = i / words_per_row;
    const int64_t word = i - row * words_per_row;
    const int64_t bit0 = word * 32;
    const int64_t v0 = bit0 / bits;
    const int64_t v1 = (bit0 + 31) / bits;
    uint32_t out = 0;
    for (int64_t v = v0; v <= v1; ++v) {
      const uint32_t code = rng_code(seed, uint64_t(row * k + v), bits);
      const int64_t sh = v * bits - bit0;
      out |= sh >= 0 ? (code << sh) : (code >> (-sh));
    }
    dst[i] = out;
  }
}

__global__ void eval_math_kernel(int op, const float* __restrict__ in, float* __restrict__ out,
                                 int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    const float v = in[i];
    float r;
    switch (op) {
      case 0: r = expf_(v); break;
      case 1: r = log1pf_(v); break;
      case 2: r = sigmoidf_(v); break;
      case 3: r = softplusf_(v); break;
      default: r = round_bf16(v); break;
    }
    out[i] = r;
  }
}

// Zero-mean affine groups: b = bf16(-s * (2^bits - 1) / 2 + U(-noise, noise)),
// so that the dequantised weights s*q + b of uniform codes centre on zero.
__global__ void fill_bias_centered_kernel(uint16_t* __restrict__ b, const uint16_t* __restrict__ s,
                                          size_t count, int bits, uint64_t seed, float noise) {
  const float mid = float((1u << bits) - 1u) * 0.5f;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += size_t(gridDim.x) * blockDim.x)
    b[i] = f32_to_bf16(fmaf_(-bf16_to_f32(s[i]), mid, rng_uniform(seed, i, -noise, noise)));
}

__global__ void fill_f32_kernel(float* __restrict__ dst, size_t count, uint64_t seed, float a,
                                float b) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += size_t(gridDim.x) * blockDim.x)
    dst[i] = rng_uniform(seed, i, a, b);
}

int grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return int(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

}  // namespace

int fill_bf16(uint16_t* dst, size_t count, uint64_t seed, int dist, float a, float b,
              hipStream_t s) {
  if (count == 0) return MX_OK;
  hipLaunchKernelGGL(fill_bf16_kernel, dim3(grid_for(int64_t(count))), dim3(256), 0, s, dst, count,
                     seed, dist, a, b);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int fill_codes(uint32_t* dst, int64_t rows, int k, int bits, uint64_t seed, hipStream_t s) {
  const int64_t words = (rows * k * bits) >> 5;
  if (words == 0) return MX_OK;
  hipLaunchKernelGGL(fill_codes_kernel, dim3(grid_for(words)), dim3(256), 0, s, dst, rows, k, bits,
                     seed);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int fill_bias_centered(uint16_t* b, const uint16_t* scales, size_t count, int bits, uint64_t seed,
                       float noise, hipStream_t s) {
  if (count == 0) return MX_OK;
  hipLaunchKernelGGL(fill_bias_centered_kernel, dim3(grid_for(int64_t(count))), dim3(256), 0, s, b,
                     scales, count, bits, seed, noise);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int fill_f32(float* dst, size_t count, uint64_t seed, float a, float b, hipStream_t s) {
  if (count == 0) return MX_OK;
  hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(int64_t(count))), dim3(256), 0, s, dst, count,
                     seed, a, b);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int eval_math(int op, const float* in, float* out, int64_t n, hipStream_t s) {
  if (n == 0) return MX_OK;
  hipLaunchKernelGGL(eval_math_kernel, dim3(grid_for(n)), dim3(256), 0, s, op, in, out, n);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
