/*
 * core.c — scalar arithmetic, generator and affine quantisation restated.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float mxo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Round to nearest even; NaN -> quiet NaN with the sign kept. */
uint16_t mxo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(0x7fc0u | ((u >> 16) & 0x8000u));
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float rbf(float f) { return mxo_bf16_to_f32(mxo_f32_to_bf16(f)); }

/* e^x by Cody-Waite reduction (ln2 split 0.693145751953125 + 1.4286068e-6)
 * and the degree-7 Taylor polynomial of e^r, scaled by 2^n. */
float mxo_expf(float x) {
  if (isnan(x)) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.972084045410156f) return 0.0f;
  const float t = x * 1.44269502162933349609375f;
  const float n = rintf(t);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698e-04f;
  p = fmaf(p, r, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333377e-03f);
  p = fmaf(p, r, 4.16666679e-02f);
  p = fmaf(p, r, 1.66666672e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) {
    p = p * 2.0f;
    ni -= 1;
  }
  if (ni < -126) {
    p = p * u2f((uint32_t)(ni + 64 + 127) << 23);
    return p * 5.42101086242752217004e-20f;
  }
  return p * u2f((uint32_t)(ni + 127) << 23);
}

/* log(1+u): atanh series of the mantissa in [sqrt(1/2), sqrt(2)) plus e*ln2,
 * with a first-order correction for the rounding of 1+u. */
float mxo_log1pf(float u) {
  if (isnan(u)) return u;
  if (isinf(u) && u > 0) return u;
  const float w = 1.0f + u;
  if (w == 1.0f) return u;
  if (w <= 0.0f) return w == 0.0f ? -INFINITY : NAN;
  const uint32_t bits = f2u(w);
  int e = (int)((bits >> 23) & 0xff) - 127;
  float m = u2f((bits & 0x007fffffu) | 0x3f800000u);
  if (m > 1.41421353816986083984375f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  float p = 0.1818181818f;
  p = fmaf(p, z, 0.2222222222f);
  p = fmaf(p, z, 0.2857142857f);
  p = fmaf(p, z, 0.4f);
  p = fmaf(p, z, 0.6666666667f);
  p = fmaf(p, z, 2.0f);
  const float fe = (float)e;
  float lg = fmaf(s, p, fe * 1.428606765330187045e-06f);
  lg = fmaf(fe, 0.693145751953125f, lg);
  const float corr = (u - (w - 1.0f)) / w;
  return lg + corr;
}

/* MLX Sigmoid form (reference kernels/moe_route_tail.metal:119-123):
 * y = 1/(1+e^|x|); x<0 ? y : 1-y. */
float mxo_sigmoidf(float x) {
  const float y = 1.0f / (1.0f + mxo_expf(fabsf(x)));
  return x < 0.0f ? y : 1.0f - y;
}

/* logaddexp(x, 0) as in compiled::decay (reference src/compiled.rs:15). */
float mxo_softplusf(float x) {
  const float m = x > 0.0f ? x : 0.0f;
  return m + mxo_log1pf(mxo_expf(-fabsf(x)));
}

void mxo_eval_math(int op, const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = in[i];
    switch (op) {
      case 0: out[i] = mxo_expf(v); break;
      case 1: out[i] = mxo_log1pf(v); break;
      case 2: out[i] = mxo_sigmoidf(v); break;
      case 3: out[i] = mxo_softplusf(v); break;
      default: out[i] = rbf(v); break;
    }
  }
}

/* ---- generator: SplitMix64 finaliser applied to seed + (idx+1)*golden ---- */
static uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
uint64_t mxo_rng_u64(uint64_t seed, uint64_t idx) {
  return mix64(seed + (idx + 1ull) * 0x9e3779b97f4a7c15ull);
}
static float rng_normal(uint64_t seed, uint64_t idx) {
  const uint64_t s2 = seed ^ 0x6a09e667f3bcc909ull;
  int32_t acc = 0;
  for (int j = 0; j < 3; ++j) {
    const uint64_t r = mxo_rng_u64(s2, idx * 3ull + (uint64_t)j);
    acc += (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) +
           (int32_t)((r >> 48) & 0xffff);
  }
  return (float)(acc - 393210) * 1.52587890625e-05f;
}
void mxo_fill_bf16(uint16_t* dst, size_t count, uint64_t seed, int dist, float a, float b) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)count; ++i) {
    float v;
    if (dist == 0) {
      const float u = (float)(uint32_t)(mxo_rng_u64(seed, (uint64_t)i) >> 40) * 5.9604644775390625e-08f;
      v = fmaf(u, b - a, a);
    } else {
      v = fmaf(rng_normal(seed, (uint64_t)i), a, b);
    }
    dst[i] = mxo_f32_to_bf16(v);
  }
}
/* Codes in MLX layout: value v of row r is code(seed, r*k+v), stored at bit
 * v*bits of the row's little-endian bitstream. */
void mxo_fill_codes(uint32_t* dst, int64_t rows, int k, int bits, uint64_t seed) {
  const int64_t wpr = ((int64_t)k * bits) >> 5;
  memset(dst, 0, (size_t)(rows * wpr) * 4);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    uint32_t* row = dst + r * wpr;
    for (int v = 0; v < k; ++v) {
      const uint32_t code = (uint32_t)(mxo_rng_u64(seed, (uint64_t)(r * k + v)) >> (64 - bits));
      const int64_t bit = (int64_t)v * bits;
      const int64_t w = bit >> 5;
      const int off = (int)(bit & 31);
      row[w] |= code << off;
      if (off + bits > 32) row[w + 1] |= code >> (32 - off);
    }
  }
}

/* Value k of a row: bits [k*bits, k*bits+bits) of the little-endian
 * bitstream (reference kernels/verify_qmv.h:60-116 byte masks; for 5 bits
 * eight values per five bytes, for 6 bits four values per three bytes). */
uint32_t mxo_code(const uint32_t* row_words, int k, int bits) {
  const int64_t bit = (int64_t)k * bits;
  const int64_t w = bit >> 5;
  const int off = (int)(bit & 31);
  uint32_t v = row_words[w] >> off;
  if (off + bits > 32) v |= row_words[w + 1] << (32 - off);
  return v & ((1u << bits) - 1u);
}

/* ops::dequantize (reference src/weights.rs:216-222): w = s*q + b in fp32,
 * rounded to bf16; s*q is exact so mul+add and fma agree. */
void mxo_dequant_rows(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                      int n, int k, int bits, int gs, const uint32_t* ids, int count,
                      uint16_t* out) {
  const int64_t wpr = ((int64_t)k * bits) >> 5;
  const int gpr = k / gs;
  for (int i = 0; i < count; ++i) {
    const int64_t row = ids[i] < (uint32_t)n ? ids[i] : (uint32_t)(n - 1);
    for (int c = 0; c < k; ++c) {
      const float q = (float)mxo_code(codes + row * wpr, c, bits);
      const float s = mxo_bf16_to_f32(scales[row * gpr + c / gs]);
      const float b = mxo_bf16_to_f32(biases[row * gpr + c / gs]);
      out[(int64_t)i * k + c] = mxo_f32_to_bf16(s * q + b);
    }
  }
}

static int lanes_per_row(int k) {
  const int chunks = k / 32;
  int L = 1;
  while (L * 2 <= chunks && L < 64) L *= 2;
  return L;
}

/* One output row of the affine QMV before the final bf16 rounding, restating
 * MLX's  s*sum(x q) + b*sum(x)  per group (reference kernels/verify_qmv.h:112,
 * verify_qmv.metal:30-64) in the build's fixed order: 32-value chunks (fma
 * chain over j from +0, sequential sum of x), per-chunk fma(s, acc, b*sx),
 * lane l of L sums chunks c = l mod L in ascending order, xor butterfly over
 * the L lanes (offsets L/2 .. 1).  L depends on k only, so the value of a row
 * never depends on how many activation rows share the weight stream. */
float mxo_qmv_row(const uint32_t* rw, const uint16_t* srow, const uint16_t* brow, int k, int bits,
                  int gs, const uint16_t* xr) {
  const int chunks = k / 32;
  const int L = lanes_per_row(k);
  float lane[64], tmp[64];
  for (int l = 0; l < L; ++l) lane[l] = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    float acc = 0.0f, sx = 0.0f;
    for (int j = 0; j < 32; ++j) {
      const float xv = mxo_bf16_to_f32(xr[32 * c + j]);
      const float q = (float)mxo_code(rw, 32 * c + j, bits);
      acc = fmaf(xv, q, acc);
      sx = sx + xv;
    }
    const int g = (32 * c) / gs;
    const float s = mxo_bf16_to_f32(srow[g]);
    const float b = mxo_bf16_to_f32(brow[g]);
    lane[c % L] = lane[c % L] + fmaf(s, acc, b * sx);
  }
  for (int o = L >> 1; o > 0; o >>= 1) {
    for (int l = 0; l < L; ++l) tmp[l] = lane[l] + lane[l ^ o];
    for (int l = 0; l < L; ++l) lane[l] = tmp[l];
  }
  return lane[0];
}

void mxo_qmv(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n, int k,
             int bits, int gs, const uint16_t* x, int m, uint16_t* y) {
  const int64_t wpr = ((int64_t)k * bits) >> 5;
  const int gpr = k / gs;
#pragma omp parallel for schedule(static)
  for (int row = 0; row < n; ++row) {
    for (int mm = 0; mm < m; ++mm)
      y[(int64_t)mm * n + row] =
          mxo_f32_to_bf16(mxo_qmv_row(codes + (int64_t)row * wpr, scales + (int64_t)row * gpr,
                                      biases + (int64_t)row * gpr, k, bits, gs, x + (int64_t)mm * k));
  }
}

/* Closed form in double: sum_k x_k (s q_k + b), no rounding until the end. */
void mxo_qmv_f64(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n,
                 int k, int bits, int gs, const uint16_t* x, int m, double* y) {
  const int64_t wpr = ((int64_t)k * bits) >> 5;
  const int gpr = k / gs;
#pragma omp parallel for schedule(static)
  for (int row = 0; row < n; ++row) {
    const uint32_t* rw = codes + (int64_t)row * wpr;
    for (int mm = 0; mm < m; ++mm) {
      double acc = 0.0;
      for (int c = 0; c < k; ++c) {
        const double s = mxo_bf16_to_f32(scales[(int64_t)row * gpr + c / gs]);
        const double b = mxo_bf16_to_f32(biases[(int64_t)row * gpr + c / gs]);
        acc += (double)mxo_bf16_to_f32(x[(int64_t)mm * k + c]) * (s * mxo_code(rw, c, bits) + b);
      }
      y[(int64_t)mm * n + row] = acc;
    }
  }
}

int mxo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
