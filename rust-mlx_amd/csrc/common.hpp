// Shared helpers for the gfx950 kernels and the host engine: bf16 rounding,
// deterministic transcendental functions, the counter-based generator, and
// error plumbing for the C ABI.
//
// Determinism contract: every floating-point step below uses only IEEE
// single-precision add/mul/div/sqrt and explicit fused multiply-adds, and the
// library is compiled with -ffp-contract=off.  The same arithmetic therefore
// yields the same bits on the GPU and in a CPU restatement that performs the
// same operations in the same order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MX_HD __host__ __device__ __forceinline__

namespace mx {

MX_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
MX_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// bf16 -> fp32 is exact.
MX_HD float bf16_to_f32(uint16_t h) { return u2f(uint32_t(h) << 16); }

// fp32 -> bf16, round to nearest even; NaN becomes the canonical quiet NaN.
// (Written as selects: no branch on the device.)
MX_HD uint16_t f32_to_bf16(float f) {
  const uint32_t u = f2u(f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t q = 0x7fc0u | ((u >> 16) & 0x8000u);
  return uint16_t((u & 0x7fffffffu) > 0x7f800000u ? q : r);
}

// Round an fp32 value to the nearest bf16 value, keeping fp32 storage.
MX_HD float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

MX_HD float fmaf_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// e^x: Cody-Waite reduction x = n*ln2 + r, |r| <= ln2/2, degree-7 Taylor
// polynomial for e^r, then exact scaling by 2^n (two steps below 2^-126).
// Branch-free: the reduction runs on x clamped to [-104, 89] (a no-op inside
// the finite range), and NaN, overflow (x > 88.7228...: +inf) and underflow
// (x < -103.972...: 0) are selected at the end; the same bits as handling
// them first, for every fp32 input.
MX_HD float expf_(float x) {
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);
  const float t = xc * 1.44269502162933349609375f;
  const float n = __builtin_rintf(t);
  float r = fmaf_(-n, 0.693145751953125f, xc);
  r = fmaf_(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698e-04f;          // 1/5040
  p = fmaf_(p, r, 1.38888889e-03f);   // 1/720
  p = fmaf_(p, r, 8.33333377e-03f);   // 1/120
  p = fmaf_(p, r, 4.16666679e-02f);   // 1/24
  p = fmaf_(p, r, 1.66666672e-01f);   // 1/6
  p = fmaf_(p, r, 0.5f);
  p = fmaf_(p, r, 1.0f);
  p = fmaf_(p, r, 1.0f);
  int ni = int(n);
  const bool big = ni > 127;
  p = big ? p * 2.0f : p;
  ni = big ? ni - 1 : ni;
  const float lo = (p * u2f(uint32_t(ni + 64 + 127) << 23)) * 5.42101086242752217004e-20f;  // 2^-64
  const float hi = p * u2f(uint32_t(ni + 127) << 23);
  float res = ni < -126 ? lo : hi;
  res = x > 88.72283935546875f ? u2f(0x7f800000u) : res;
  res = x < -103.972084045410156f ? 0.0f : res;
  return x != x ? x : res;
}

// bf16 logistic function with MLX's per-operation bf16 rounding
// (reference kernels/moe_route_tail.metal:119-123).
__device__ __forceinline__ float sigmoid_bf16(float x) {
  const float e = round_bf16(expf_(__builtin_fabsf(x)));
  const float d = round_bf16(1.0f + e);
  const float y = round_bf16(1.0f / d);
  return x < 0.0f ? y : round_bf16(1.0f - y);
}

// log(1 + u) for u > -1: w = 1 + u split as m * 2^e with m in [sqrt(1/2),
// sqrt(2)); log m from the atanh series in s = (m-1)/(m+1); first-order
// correction for the rounding of w.
MX_HD float log1pf_(float u) {
  if (u != u) return u;
  if (u == u2f(0x7f800000u)) return u;
  const float w = 1.0f + u;
  if (w == 1.0f) return u;
  if (w <= 0.0f) return w == 0.0f ? u2f(0xff800000u) : u2f(0x7fc00000u);
  uint32_t bits = f2u(w);
  int e = int((bits >> 23) & 0xff) - 127;
  float m = u2f((bits & 0x007fffffu) | 0x3f800000u);
  if (m > 1.41421353816986083984375f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  float p = 0.1818181818f;       // 2/11
  p = fmaf_(p, z, 0.2222222222f);  // 2/9
  p = fmaf_(p, z, 0.2857142857f);  // 2/7
  p = fmaf_(p, z, 0.4f);           // 2/5
  p = fmaf_(p, z, 0.6666666667f);  // 2/3
  p = fmaf_(p, z, 2.0f);
  const float fe = float(e);
  float lg = fmaf_(s, p, fe * 1.428606765330187045e-06f);
  lg = fmaf_(fe, 0.693145751953125f, lg);
  const float corr = (u - (w - 1.0f)) / w;
  return lg + corr;
}

// Logistic function in the form MLX's Sigmoid uses: y = 1 / (1 + e^|x|),
// sigma(x) = y for x < 0 and 1 - y otherwise.
MX_HD float sigmoidf_(float x) {
  const float y = 1.0f / (1.0f + expf_(__builtin_fabsf(x)));
  return x < 0.0f ? y : 1.0f - y;
}

// softplus(x) = logaddexp(x, 0) = max(x, 0) + log1p(e^-|x|).
MX_HD float softplusf_(float x) {
  const float m = x > 0.0f ? x : 0.0f;
  return m + log1pf_(expf_(-__builtin_fabsf(x)));
}

// ---- counter-based generator (SplitMix64 finaliser over seed + counter) ----
MX_HD uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
MX_HD uint64_t rng_u64(uint64_t seed, uint64_t idx) {
  return mix64(seed + (idx + 1ull) * 0x9e3779b97f4a7c15ull);
}
// U[0,1) with 24 random bits (exact in fp32).
MX_HD float rng_unit(uint64_t seed, uint64_t idx) {
  return float(uint32_t(rng_u64(seed, idx) >> 40)) * 5.9604644775390625e-08f;
}
MX_HD float rng_uniform(uint64_t seed, uint64_t idx, float a, float b) {
  return fmaf_(rng_unit(seed, idx), b - a, a);
}
// Approximately N(0,1): Irwin-Hall sum of twelve 16-bit uniforms, centred and
// scaled by 2^-16 (every step exact, so CPU and GPU agree bit for bit).
MX_HD float rng_normal(uint64_t seed, uint64_t idx) {
  const uint64_t s2 = seed ^ 0x6a09e667f3bcc909ull;
  int32_t acc = 0;
  for (int j = 0; j < 3; ++j) {
    const uint64_t r = rng_u64(s2, idx * 3ull + uint64_t(j));
    acc += int32_t(r & 0xffff) + int32_t((r >> 16) & 0xffff) + int32_t((r >> 32) & 0xffff) +
           int32_t((r >> 48) & 0xffff);
  }
  return float(acc - 393210) * 1.52587890625e-05f;
}
// Code of value `idx` for a `bits`-bit uniform integer stream.
MX_HD uint32_t rng_code(uint64_t seed, uint64_t idx, int bits) {
  return uint32_t(rng_u64(seed, idx) >> (64 - bits));
}

}  // namespace mx

// ---- host-side error plumbing (defined in capi.cpp) ----
#include <string>

#include "../../include/mx355.h"
namespace mx {
int set_error(int code, const std::string& msg);
int hip_error(hipError_t e, const char* what);
}  // namespace mx
#define MX_HIP(call)                                               \
  do {                                                             \
    hipError_t e_ = (call);                                        \
    if (e_ != hipSuccess) return mx_status(mx::hip_error(e_, #call));      \
  } while (0)
#define MX_CHECK(cond, code, msg)                                  \
  do {                                                             \
    if (!(cond)) return mx_status(mx::set_error((code), (msg)));            \
  } while (0)
