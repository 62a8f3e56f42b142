/* Exact-integer affine projection (XQ): the arithmetic of the engine's
 * bit-exact product path, restated on the CPU.  TEST INFRASTRUCTURE ONLY.
 *
 * The affine projection of reference kernels/verify_qmv.h:112
 * (s * sum(x q) + b * sum(x) per group, MLX's affine layout) with the sums
 * made exact, so that no summation order is left to define:
 *
 *  - per 64-value group g of an activation row, let Eb be the largest bf16
 *    exponent field among the group's values (at least 1); every value x_k
 *    (sign, exponent field e_k, significand m_k with the hidden bit, e_k = 0
 *    read as 1) becomes the integer X_k = sign * floor(m_k 2^(e_k - Eb + 22)),
 *    i.e. x_k on the grid 2^(Eb - 156), truncated toward zero when
 *    e_k < Eb - 22 (|X_k| < 2^30);
 *  - P = sum_k X_k q_k and Q = sum_k X_k are exact integers (|P| < 2^44);
 *  - the group's value is v_g = fma(P, s_g, Q b_g) * 2^(Eb - 156) in double
 *    (P s_g and Q b_g are exact products; one rounding in the fma);
 *  - the groups are added in double, in order, within each slice of two
 *    consecutive groups (the last slice of an odd count holds one), each
 *    slice sum starting from +0; the slice sums are added in order from +0;
 *    the total is rounded once to fp32.
 *
 * On the GPU the integer sums are int8 matrix-core products of the signed
 * base-256 digits of X_k with the codes (exact in int32), so the result
 * does not depend on how the hardware orders a sum.  Group size 64 only. */
#include <math.h>
#include <stdint.h>

#include "oracle.h"

int mxo_xq_slices(int k) { return (k / 64 + 1) / 2; }

/* X_k of one bf16 value on the grid of exponent field eb. */
int64_t mxo_xq_int(uint16_t h, int eb) {
  const int e = (h >> 7) & 0xff;
  const int64_t mant = (e ? 0x80 : 0) | (h & 0x7f);
  const int sh = (e ? e : 1) - eb + 22;
  const int64_t v = sh >= 0 ? (mant << sh) : (sh > -8 ? (mant >> -sh) : 0);
  return (h & 0x8000) ? -v : v;
}

/* Largest exponent field of a 64-value group (at least 1). */
int mxo_xq_group_exp(const uint16_t* x) {
  int eb = 1;
  for (int j = 0; j < 64; ++j) {
    const int e = (x[j] >> 7) & 0xff;
    if (e > eb) eb = e;
  }
  return eb;
}

float mxo_xq_row(const uint32_t* rw, const uint16_t* srow, const uint16_t* brow, int k, int bits,
                 const uint16_t* x) {
  const int G = k / 64, S = mxo_xq_slices(k);
  double total = 0.0;
  for (int sl = 0; sl < S; ++sl) {
    double acc = 0.0;
    for (int g = 2 * sl; g < 2 * sl + 2 && g < G; ++g) {
      const int eb = mxo_xq_group_exp(x + 64 * g);
      int64_t P = 0, Q = 0;
      for (int j = 0; j < 64; ++j) {
        const int64_t X = mxo_xq_int(x[64 * g + j], eb);
        P += X * (int64_t)mxo_code(rw, 64 * g + j, bits);
        Q += X;
      }
      const double s = mxo_bf16_to_f32(srow[g]), b = mxo_bf16_to_f32(brow[g]);
      const double v = fma((double)P, s, (double)Q * b);
      acc = acc + ldexp(v, eb - 156);
    }
    total = total + acc;
  }
  return (float)total;
}

void mxo_xq(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n, int k,
            int bits, const uint16_t* x, int m, float* y) {
  const int64_t wpr = ((int64_t)k * bits) >> 5;
  const int gpr = k / 64;
#pragma omp parallel for schedule(static)
  for (int row = 0; row < n; ++row)
    for (int mm = 0; mm < m; ++mm)
      y[(int64_t)mm * n + row] = mxo_xq_row(codes + (int64_t)row * wpr, scales + (int64_t)row * gpr,
                                            biases + (int64_t)row * gpr, k, bits, x + (int64_t)mm * k);
}
