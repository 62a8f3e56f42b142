// Device core of every affine-quantised projection (plain QMV, gathered
// experts, vocabulary head).  One lane group of L lanes computes R output rows
// for M activation rows in the library's fixed order:
//   * K is cut into 32-value chunks; lane l of the group owns chunks
//     c = l, l+L, l+2L, ... (ascending);
//   * per chunk: acc = fma chain over j = 0..31 of x*q (from +0), sx = sequential
//     fp32 sum of x, part = fma(scale, acc, bias * sx)  — MLX's
//     s*sum(xq) + b*sum(x) per group (reference kernels/verify_qmv.h:112);
//   * lane sums add parts in chunk order from +0; an xor butterfly over the L
//     lanes (offsets L/2 .. 1) finishes the row.
// L = min(64, largest power of two <= K/32) depends on K only, so batching rows
// (M) or gathering experts never changes a result's bits.
#pragma once

#include "common.hpp"

namespace mx {

constexpr int kQRows = 4;  // output rows per lane group

__host__ __device__ inline int qmv_lanes_per_row(int k) {
  const int chunks = k / 32;
  int L = 1;
  while (L * 2 <= chunks && L < 64) L *= 2;
  return L;
}

template <int BITS>
__device__ __forceinline__ void qload_chunk(const uint32_t* __restrict__ p, uint32_t (&w)[BITS]) {
  if constexpr (BITS == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (BITS == 8) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (BITS == 6) {
    const uint2 a = *reinterpret_cast<const uint2*>(p);
    const uint2 b = *reinterpret_cast<const uint2*>(p + 2);
    const uint2 c = *reinterpret_cast<const uint2*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y; w[4] = c.x; w[5] = c.y;
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = p[i];
  }
}

// All 32 codes of a chunk as exact floats, value j at bit j*BITS.
template <int BITS>
__device__ __forceinline__ void qunpack(const uint32_t (&w)[BITS], float (&q)[32]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = w[i] & 0x0f0f0f0fu;         // values 0,2,4,6 of the word
      const uint32_t hi = (w[i] >> 4) & 0x0f0f0f0fu;  // values 1,3,5,7
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        q[8 * i + 2 * b] = float((lo >> (8 * b)) & 0xffu);
        q[8 * i + 2 * b + 1] = float((hi >> (8 * b)) & 0xffu);
      }
    }
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int b = 0; b < 4; ++b) q[4 * i + b] = float((w[i] >> (8 * b)) & 0xffu);
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int bit = j * BITS;
      const int word = bit >> 5;
      const int off = bit & 31;
      uint32_t v = w[word] >> off;
      if (off + BITS > 32) v |= w[word + 1] << (32 - off);
      q[j] = float(v & ((1u << BITS) - 1u));
    }
  }
}

__device__ __forceinline__ float xval(const uint32_t (&xw)[16], int j) {
  const uint32_t d = xw[j >> 1];
  return (j & 1) ? u2f(d & 0xffff0000u) : u2f(d << 16);
}

// Computes out[m][r] = sum over this lane group of rows rows[r] for activation
// rows xrow[m] (M of them).  Every lane of the group ends with the full sums.
// `rows` must be valid (in-bounds) row indices.
template <int BITS, int M>
__device__ __forceinline__ void qmv_core(const uint32_t* __restrict__ codes,
                                         const uint16_t* __restrict__ scales,
                                         const uint16_t* __restrict__ biases, int k, int gs,
                                         const uint16_t* const (&xrow)[M], const int (&rows)[kQRows],
                                         int li, int L, float (&out)[M][kQRows]) {
  const int chunks = k >> 5;
  const int words_per_row = (k * BITS) >> 5;
  const int groups_per_row = k / gs;
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < kQRows; ++r) out[m][r] = 0.0f;

  for (int c = li; c < chunks; c += L) {
    uint32_t xw[M][16];
    float sx[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* xp = reinterpret_cast<const uint4*>(xrow[m] + size_t(c) * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = xp[q];
        xw[m][4 * q + 0] = v.x; xw[m][4 * q + 1] = v.y;
        xw[m][4 * q + 2] = v.z; xw[m][4 * q + 3] = v.w;
      }
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) s = s + xval(xw[m], j);
      sx[m] = s;
    }
    const int g = (c * 32) / gs;
#pragma unroll
    for (int r = 0; r < kQRows; ++r) {
      uint32_t w[BITS];
      qload_chunk<BITS>(codes + size_t(rows[r]) * words_per_row + size_t(c) * BITS, w);
      const float sc = bf16_to_f32(scales[size_t(rows[r]) * groups_per_row + g]);
      const float bi = bf16_to_f32(biases[size_t(rows[r]) * groups_per_row + g]);
      float q[32];
      qunpack<BITS>(w, q);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) acc = fmaf_(xval(xw[m], j), q[j], acc);
        out[m][r] = out[m][r] + fmaf_(sc, acc, bi * sx[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < kQRows; ++r) {
      float v = out[m][r];
      for (int o = L >> 1; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
      out[m][r] = v;
    }
}

}  // namespace mx
