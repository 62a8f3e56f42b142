// Matrix-core core of the fast affine-quantised projections (gfx950 MFMA).
//
// y[m, n] = sum_g s[n,g] * sum_{k in g} x[m,k] q[n,k] + b[n,g] * sum_{k in g} x[m,k]
// for up to 16 activation rows m against 16-row weight tiles n, group size 64.
//
// One v_mfma_f32_16x16x32_bf16 multiplies A (16 activation rows x 32 k) by
// B (32 k x 16 weight rows).  Lane l holds A row l%16 and B column l%16 for
// k = 8*(l/16) .. +7 of the step, and receives D rows 4*(l/16) .. +3 of
// column l%16.  Within a 64-value group, lane quarter kq = l/16 covers values
// 16*kq .. +15 in two steps of 8, so each MFMA sums one group only; the
// group's scale and bias are then applied to the fp32 partial in registers.
//
// Codes enter the matrix core as exact bf16 integers: for widths <= 7 bits,
// (0x4300 | q) is the bf16 value 128 + q (one bit operation per pair); the
// 128 * sum(x) this adds is removed through the bias (b - 128 s).  8-bit codes
// are converted exactly through fp32.  Within each 8-value unit the k order is
// (0,4,1,5,2,6,3,7) on both operands, matching how nibble pairs are split.
//
// Arithmetic is dequantise-free: products x*q are exact, sums are fp32 inside
// the matrix core (hardware order), then s * acc + (b - off*s) * sum(x) in fp32.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace mx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma_bf16(const uint4& a, const uint4& b, floatx4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// x values [v0..v7] as packed bf16 pairs (v0v1, v2v3, v4v5, v6v7) ->
// operand order (v0, v4, v1, v5, v2, v6, v3, v7).
__device__ __forceinline__ uint4 permute_x(const uint4& x) {
  uint4 r;
  r.x = __builtin_amdgcn_perm(x.z, x.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(x.z, x.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(x.w, x.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(x.w, x.y, 0x07060302u);
  return r;
}

// Offset the code encoding adds to every value (128 for <= 7 bits, 0 for 8).
template <int BITS>
constexpr float code_offset() {
  return BITS == 8 ? 0.0f : 128.0f;
}

// Words of packed codes each lane loads per 64-value group.
template <int BITS>
constexpr int group_words() {
  return BITS == 4 ? 2 : BITS == 5 ? 3 : BITS == 6 ? 3 : 4;
}

// Loads lane quarter kq's 16 codes of group g of a row into `w`, normalised so
// that value v starts at bit BITS*v of (w[0], w[1], ...).
template <int BITS>
__device__ __forceinline__ void load_group_codes(const uint32_t* __restrict__ row, int g, int kq,
                                                 uint32_t (&w)[group_words<BITS>()]) {
  if constexpr (BITS == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + 8 * g + 2 * kq);
    w[0] = v.x;
    w[1] = v.y;
  } else if constexpr (BITS == 5) {
    const int bit = 80 * kq;  // within the group's 320 bits (10 words)
    const uint32_t* p = row + 10 * g + (bit >> 5);
    const uint32_t a = p[0], b = p[1], c = p[2];
    const uint32_t sh = uint32_t(bit & 31);  // 0 or 16
    w[0] = __builtin_amdgcn_alignbit(b, a, sh);
    w[1] = __builtin_amdgcn_alignbit(c, b, sh);
    w[2] = sh ? (c >> 16) : c;
  } else if constexpr (BITS == 6) {
    const uint32_t* p = row + 12 * g + 3 * kq;
    w[0] = p[0];
    w[1] = p[1];
    w[2] = p[2];
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(row + 16 * g + 4 * kq);
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
  }
}

template <int BITS, int V>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&w)[group_words<BITS>()]) {
  constexpr int bit = BITS * V;
  constexpr int word = bit >> 5;
  constexpr int off = bit & 31;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if constexpr (off + BITS <= 32) {
    return (w[word] >> off) & mask;
  } else {
    return __builtin_amdgcn_alignbit(w[word + 1], w[word], uint32_t(off)) & mask;
  }
}

// B operand for step t (values 8t .. 8t+7) in operand order.
template <int BITS, int T>
__device__ __forceinline__ uint4 codes_operand(const uint32_t (&w)[group_words<BITS>()]) {
  uint4 r;
  if constexpr (BITS == 4) {
    const uint32_t x = w[T];
    r.x = (x & 0x000F000Fu) | 0x43004300u;
    r.y = ((x >> 4) & 0x000F000Fu) | 0x43004300u;
    r.z = ((x >> 8) & 0x000F000Fu) | 0x43004300u;
    r.w = ((x >> 12) & 0x000F000Fu) | 0x43004300u;
  } else if constexpr (BITS == 8) {
    // bytes (v0..v3) in w[2T], (v4..v7) in w[2T+1]; exact through fp32
    const uint32_t lo = w[2 * T], hi = w[2 * T + 1];
    auto pair = [](float a, float b) {
      return __builtin_amdgcn_perm(f2u(b), f2u(a), 0x07060302u);
    };
    // float(byte) compiles to v_cvt_f32_ubyte{0..3}
    r.x = pair(float(lo & 0xffu), float(hi & 0xffu));
    r.y = pair(float((lo >> 8) & 0xffu), float((hi >> 8) & 0xffu));
    r.z = pair(float((lo >> 16) & 0xffu), float((hi >> 16) & 0xffu));
    r.w = pair(float(lo >> 24), float(hi >> 24));
  } else {
    r.x = (code_at<BITS, 8 * T + 0>(w) | (code_at<BITS, 8 * T + 4>(w) << 16)) | 0x43004300u;
    r.y = (code_at<BITS, 8 * T + 1>(w) | (code_at<BITS, 8 * T + 5>(w) << 16)) | 0x43004300u;
    r.z = (code_at<BITS, 8 * T + 2>(w) | (code_at<BITS, 8 * T + 6>(w) << 16)) | 0x43004300u;
    r.w = (code_at<BITS, 8 * T + 3>(w) | (code_at<BITS, 8 * T + 7>(w) << 16)) | 0x43004300u;
  }
  return r;
}

// One weight tile's row (this lane's row l%16) as plain pointers.
struct TileRow {
  const uint32_t* codes;   // the row's packed codes
  const uint16_t* scales;  // the row's K/64 scales
  const uint16_t* biases;
};

__device__ __forceinline__ TileRow tile_row(const uint32_t* codes, const uint16_t* scales,
                                            const uint16_t* biases, int k, int bits, int row) {
  const int wpr = (k * bits) >> 5;
  const int G = k >> 6;
  return TileRow{codes + size_t(row) * wpr, scales + size_t(row) * G, biases + size_t(row) * G};
}

// Accumulates groups [g0, g1) of NT weight tiles into y[nt] (D layout: lane l
// holds activation rows 4*(l/16)+r of tile row l%16).  `xa` is this lane's
// activation row (lane%16), or nullptr when that row is beyond M (zero A).
// Groups are processed in batches of four: every load of a batch is issued
// before any of its matrix-core work, so each wave keeps several memory round
// trips in flight.  The group sums of x come from one more MFMA against a
// ones operand (D rows = row sums), shared by the NT tiles.
template <int BITS, int NT>
__device__ __forceinline__ void qmm_tiles(const TileRow (&tr)[NT], const uint16_t* xa, int g0,
                                          int g1, floatx4_t (&y)[NT]) {
  constexpr int GB = 4;
  constexpr int NW = group_words<BITS>();
  const int lane = threadIdx.x & 63;
  const int kq = lane >> 4;
  const float off = code_offset<BITS>();
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  int g = g0;
  for (; g + GB <= g1; g += GB) {
    uint4 xv[GB][2];
    uint32_t w[GB][NT][NW];
    uint2 sc2[NT], bi2[NT];
#pragma unroll
    for (int b = 0; b < GB; ++b) {
      if (xa) {
        const uint4* xp = reinterpret_cast<const uint4*>(xa + 64 * (g + b) + 16 * kq);
        xv[b][0] = xp[0];
        xv[b][1] = xp[1];
      } else {
        xv[b][0] = xv[b][1] = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) load_group_codes<BITS>(tr[t].codes, g + b, kq, w[b][t]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // scales / biases of the four groups g .. g+3 (8 bytes each when aligned)
      if ((reinterpret_cast<uintptr_t>(tr[t].scales + g) & 7u) == 0 &&
          (reinterpret_cast<uintptr_t>(tr[t].biases + g) & 7u) == 0) {
        sc2[t] = *reinterpret_cast<const uint2*>(tr[t].scales + g);
        bi2[t] = *reinterpret_cast<const uint2*>(tr[t].biases + g);
      } else {
        sc2[t] = make_uint2(uint32_t(tr[t].scales[g]) | (uint32_t(tr[t].scales[g + 1]) << 16),
                            uint32_t(tr[t].scales[g + 2]) | (uint32_t(tr[t].scales[g + 3]) << 16));
        bi2[t] = make_uint2(uint32_t(tr[t].biases[g]) | (uint32_t(tr[t].biases[g + 1]) << 16),
                            uint32_t(tr[t].biases[g + 2]) | (uint32_t(tr[t].biases[g + 3]) << 16));
      }
    }
#pragma unroll
    for (int b = 0; b < GB; ++b) {
      const uint4 a0 = permute_x(xv[b][0]);
      const uint4 a1 = permute_x(xv[b][1]);
      floatx4_t sx = {0.0f, 0.0f, 0.0f, 0.0f};
      sx = mfma_bf16(a0, ones, sx);
      sx = mfma_bf16(a1, ones, sx);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t sw = b < 2 ? sc2[t].x : sc2[t].y;
        const uint32_t bw = b < 2 ? bi2[t].x : bi2[t].y;
        const float sc = u2f((b & 1) ? (sw & 0xffff0000u) : (sw << 16));
        const float bi = fmaf_(-off, sc, u2f((b & 1) ? (bw & 0xffff0000u) : (bw << 16)));
        floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = mfma_bf16(a0, codes_operand<BITS, 0>(w[b][t]), acc);
        acc = mfma_bf16(a1, codes_operand<BITS, 1>(w[b][t]), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) y[t][r] = fmaf_(sc, acc[r], fmaf_(bi, sx[r], y[t][r]));
      }
    }
  }
  for (; g < g1; ++g) {  // remainder groups, one at a time
    uint4 x0 = make_uint4(0, 0, 0, 0), x1 = make_uint4(0, 0, 0, 0);
    if (xa) {
      const uint4* xp = reinterpret_cast<const uint4*>(xa + 64 * g + 16 * kq);
      x0 = xp[0];
      x1 = xp[1];
    }
    const uint4 a0 = permute_x(x0), a1 = permute_x(x1);
    floatx4_t sx = {0.0f, 0.0f, 0.0f, 0.0f};
    sx = mfma_bf16(a0, ones, sx);
    sx = mfma_bf16(a1, ones, sx);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      uint32_t w[NW];
      load_group_codes<BITS>(tr[t].codes, g, kq, w);
      const float sc = bf16_to_f32(tr[t].scales[g]);
      const float bi = fmaf_(-off, sc, bf16_to_f32(tr[t].biases[g]));
      floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = mfma_bf16(a0, codes_operand<BITS, 0>(w), acc);
      acc = mfma_bf16(a1, codes_operand<BITS, 1>(w), acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) y[t][r] = fmaf_(sc, acc[r], fmaf_(bi, sx[r], y[t][r]));
    }
  }
}

// qmm_tiles for a workgroup of NTH threads whose waves all multiply the same
// 16 activation rows over the same groups [g0, g1), (g1 - g0) % 4 == 0: the
// rows pass through LDS once per batch of four groups instead of every wave
// reading them.  Thread t copies 32 bytes of row t / 16 (`xrow`, nullptr for
// a row beyond M) per batch, the next batch's piece in flight during this
// batch's work; `xs` holds one batch (16 rows of 256 values, rows padded to
// kSxLd so the lanes of one ds_read_b128 pass hit different bank groups);
// `lrow` is the row this lane's A operand takes (lane % 16), or -1 for zeros.
// Every wave of the workgroup must call it (it synchronises the workgroup).
constexpr int kSxLd = 256 + 8;

template <int BITS, int NT, int NTH>
__device__ __forceinline__ void qmm_tiles_sx(const TileRow (&tr)[NT], const uint16_t* xrow,
                                             uint16_t* xs, int lrow, int g0, int g1,
                                             floatx4_t (&y)[NT]) {
  static_assert(NTH == 256, "16 rows x 16 pieces of 32 bytes per batch");
  constexpr int GB = 4;
  constexpr int NW = group_words<BITS>();
  const int lane = threadIdx.x & 63;
  const int kq = lane >> 4;
  const float off = code_offset<BITS>();
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  const int sr = threadIdx.x >> 4, pc = threadIdx.x & 15;  // staged row, 32-byte piece
  uint4 xn0 = make_uint4(0u, 0u, 0u, 0u), xn1 = xn0;
  auto load_piece = [&](int g) {
    if (xrow) {
      const uint4* p = reinterpret_cast<const uint4*>(xrow + 64 * g + 16 * pc);
      xn0 = p[0];
      xn1 = p[1];
    }
  };
  load_piece(g0);
  for (int g = g0; g < g1; g += GB) {
    __syncthreads();  // every wave is done with the previous batch's rows
    *reinterpret_cast<uint4*>(xs + sr * kSxLd + 16 * pc) = xn0;
    *reinterpret_cast<uint4*>(xs + sr * kSxLd + 16 * pc + 8) = xn1;
    if (g + GB < g1) load_piece(g + GB);  // in flight during this batch
    uint32_t w[GB][NT][NW];
    uint2 sc2[NT], bi2[NT];
#pragma unroll
    for (int b = 0; b < GB; ++b)
#pragma unroll
      for (int t = 0; t < NT; ++t) load_group_codes<BITS>(tr[t].codes, g + b, kq, w[b][t]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if ((reinterpret_cast<uintptr_t>(tr[t].scales + g) & 7u) == 0 &&
          (reinterpret_cast<uintptr_t>(tr[t].biases + g) & 7u) == 0) {
        sc2[t] = *reinterpret_cast<const uint2*>(tr[t].scales + g);
        bi2[t] = *reinterpret_cast<const uint2*>(tr[t].biases + g);
      } else {
        sc2[t] = make_uint2(uint32_t(tr[t].scales[g]) | (uint32_t(tr[t].scales[g + 1]) << 16),
                            uint32_t(tr[t].scales[g + 2]) | (uint32_t(tr[t].scales[g + 3]) << 16));
        bi2[t] = make_uint2(uint32_t(tr[t].biases[g]) | (uint32_t(tr[t].biases[g + 1]) << 16),
                            uint32_t(tr[t].biases[g + 2]) | (uint32_t(tr[t].biases[g + 3]) << 16));
      }
    }
    __syncthreads();  // the batch's rows are in LDS
#pragma unroll
    for (int b = 0; b < GB; ++b) {
      uint4 x0 = make_uint4(0u, 0u, 0u, 0u), x1 = x0;
      if (lrow >= 0) {
        const uint4* xp = reinterpret_cast<const uint4*>(xs + lrow * kSxLd + 64 * b + 16 * kq);
        x0 = xp[0];
        x1 = xp[1];
      }
      const uint4 a0 = permute_x(x0);
      const uint4 a1 = permute_x(x1);
      floatx4_t sx = {0.0f, 0.0f, 0.0f, 0.0f};
      sx = mfma_bf16(a0, ones, sx);
      sx = mfma_bf16(a1, ones, sx);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t sw = b < 2 ? sc2[t].x : sc2[t].y;
        const uint32_t bw = b < 2 ? bi2[t].x : bi2[t].y;
        const float sc = u2f((b & 1) ? (sw & 0xffff0000u) : (sw << 16));
        const float bi = fmaf_(-off, sc, u2f((b & 1) ? (bw & 0xffff0000u) : (bw << 16)));
        floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = mfma_bf16(a0, codes_operand<BITS, 0>(w[b][t]), acc);
        acc = mfma_bf16(a1, codes_operand<BITS, 1>(w[b][t]), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) y[t][r] = fmaf_(sc, acc[r], fmaf_(bi, sx[r], y[t][r]));
      }
    }
  }
}

// The 4-bit form of qmm_tiles_sx on v_mfma_f32_32x32x16_bf16, tiles of 32
// weight rows: lane l takes weight row l % 32 and, in MFMA step s of a
// group, values 32 h + 8 s .. + 7 of it (h = l / 32) on both operands, so its
// codes of a group are 16 contiguous bytes (one load; the 16x16 form reads
// 8 bytes per lane per 16-row tile).  Activation rows 16..31 of the 32-row
// A tile are zero, so D values i < 8 (rows 8 (i / 4) + 4 h + i % 4) are the
// real ones and only they are scaled; the arithmetic per product and group
// is qmm_tiles' (fp32 sums inside the matrix core in another order).
typedef float floatx16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ floatx16_t mfma32_bf16(const uint4& a, const uint4& b, floatx16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// One 32-bit word of 8 nibble codes as a B operand in permute_x order.
__device__ __forceinline__ uint4 nibble_operand(uint32_t x) {
  uint4 r;
  r.x = (x & 0x000F000Fu) | 0x43004300u;
  r.y = ((x >> 4) & 0x000F000Fu) | 0x43004300u;
  r.z = ((x >> 8) & 0x000F000Fu) | 0x43004300u;
  r.w = ((x >> 12) & 0x000F000Fu) | 0x43004300u;
  return r;
}

// A lane's 32 codes of group g in its half h: BITS words from byte 8 BITS g +
// 4 BITS h of the row (value v at bit BITS v), in aligned 16-byte loads (4
// and 8 bits; 5 / 6-bit pieces do not start on 16-byte boundaries, and
// reading the two aligned pieces around them measured slower than the
// 16-row form).
template <int BITS>
__device__ __forceinline__ void load_half_codes(const uint32_t* __restrict__ row, int g, int h,
                                                uint32_t (&w)[BITS]) {
  static_assert(BITS == 4 || BITS == 8, "16-byte pieces");
#pragma unroll
  for (int i = 0; i < BITS / 4; ++i) {
    const uint4 v = reinterpret_cast<const uint4*>(row + 2 * BITS * g + BITS * h)[i];
    w[4 * i] = v.x;
    w[4 * i + 1] = v.y;
    w[4 * i + 2] = v.z;
    w[4 * i + 3] = v.w;
  }
}

// B operand of MFMA step s (codes 8 s .. + 7 of the lane's 32) in permute_x
// order, codes as exact bf16 integers (128 + q for 4 bits, q for 8 bits).
template <int BITS, int S>
__device__ __forceinline__ uint4 half_operand(const uint32_t (&w)[BITS]) {
  if constexpr (BITS == 4) {
    return nibble_operand(w[S]);
  } else {
    const uint32_t lo = w[2 * S], hi = w[2 * S + 1];
    auto pair = [](float a, float b) { return __builtin_amdgcn_perm(f2u(b), f2u(a), 0x07060302u); };
    uint4 r;
    r.x = pair(float(lo & 0xffu), float(hi & 0xffu));
    r.y = pair(float((lo >> 8) & 0xffu), float((hi >> 8) & 0xffu));
    r.z = pair(float((lo >> 16) & 0xffu), float((hi >> 16) & 0xffu));
    r.w = pair(float(lo >> 24), float(hi >> 24));
    return r;
  }
}

template <int BITS, int NT, int NTH>
__device__ __forceinline__ void qmm_tiles32_sx(const TileRow (&tr)[NT], const uint16_t* xrow,
                                               uint16_t* xs, int lrow, int g0, int g1,
                                               floatx16_t (&y)[NT]) {
  static_assert(NTH == 256, "16 rows x 16 pieces of 32 bytes per batch");
  constexpr int GB = 4;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5;
  const float off = code_offset<BITS>();
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  const int sr = threadIdx.x >> 4, pc = threadIdx.x & 15;
  uint4 xn0 = make_uint4(0u, 0u, 0u, 0u), xn1 = xn0;
  auto load_piece = [&](int g) {
    if (xrow) {
      const uint4* p = reinterpret_cast<const uint4*>(xrow + 64 * g + 16 * pc);
      xn0 = p[0];
      xn1 = p[1];
    }
  };
  load_piece(g0);
  for (int g = g0; g < g1; g += GB) {
    __syncthreads();  // every wave is done with the previous batch's rows
    *reinterpret_cast<uint4*>(xs + sr * kSxLd + 16 * pc) = xn0;
    *reinterpret_cast<uint4*>(xs + sr * kSxLd + 16 * pc + 8) = xn1;
    if (g + GB < g1) load_piece(g + GB);  // in flight during this batch
    uint32_t w[GB][NT][BITS];
    uint2 sc2[NT], bi2[NT];
#pragma unroll
    for (int b = 0; b < GB; ++b)
#pragma unroll
      for (int t = 0; t < NT; ++t) load_half_codes<BITS>(tr[t].codes, g + b, h, w[b][t]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if ((reinterpret_cast<uintptr_t>(tr[t].scales + g) & 7u) == 0 &&
          (reinterpret_cast<uintptr_t>(tr[t].biases + g) & 7u) == 0) {
        sc2[t] = *reinterpret_cast<const uint2*>(tr[t].scales + g);
        bi2[t] = *reinterpret_cast<const uint2*>(tr[t].biases + g);
      } else {
        sc2[t] = make_uint2(uint32_t(tr[t].scales[g]) | (uint32_t(tr[t].scales[g + 1]) << 16),
                            uint32_t(tr[t].scales[g + 2]) | (uint32_t(tr[t].scales[g + 3]) << 16));
        bi2[t] = make_uint2(uint32_t(tr[t].biases[g]) | (uint32_t(tr[t].biases[g + 1]) << 16),
                            uint32_t(tr[t].biases[g + 2]) | (uint32_t(tr[t].biases[g + 3]) << 16));
      }
    }
    __syncthreads();  // the batch's rows are in LDS
#pragma unroll
    for (int b = 0; b < GB; ++b) {
      uint4 a[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint4 xv = make_uint4(0u, 0u, 0u, 0u);
        if (lrow >= 0)
          xv = *reinterpret_cast<const uint4*>(xs + lrow * kSxLd + 64 * b + 32 * h + 8 * s);
        a[s] = permute_x(xv);
      }
      floatx16_t sx = {};
#pragma unroll
      for (int s = 0; s < 4; ++s) sx = mfma32_bf16(a[s], ones, sx);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t sw = b < 2 ? sc2[t].x : sc2[t].y;
        const uint32_t bw = b < 2 ? bi2[t].x : bi2[t].y;
        const float sc = u2f((b & 1) ? (sw & 0xffff0000u) : (sw << 16));
        const float bi = fmaf_(-off, sc, u2f((b & 1) ? (bw & 0xffff0000u) : (bw << 16)));
        floatx16_t acc = {};
        acc = mfma32_bf16(a[0], half_operand<BITS, 0>(w[b][t]), acc);
        acc = mfma32_bf16(a[1], half_operand<BITS, 1>(w[b][t]), acc);
        acc = mfma32_bf16(a[2], half_operand<BITS, 2>(w[b][t]), acc);
        acc = mfma32_bf16(a[3], half_operand<BITS, 3>(w[b][t]), acc);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[t][i] = fmaf_(sc, acc[i], fmaf_(bi, sx[i], y[t][i]));
      }
    }
  }
}

}  // namespace mx
