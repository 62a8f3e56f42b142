// Exact-integer projection core for 1..8 activation rows (gfx950,
// v_mfma_i32_16x16x64_i8), over weights in MLX's affine layout.
//
// The arithmetic (restated by the CPU oracle, oracle/xq.c):
//   per 64-value group g of activation row m, Eb = the largest bf16 exponent
//   field of the group (at least 1) and X_k = trunc(x_k 2^(156 - Eb)), an
//   integer below 2^30 in magnitude; P = sum X_k q_k and Q = sum X_k are
//   exact; v_g = fma(P, s_g, Q b_g) 2^(Eb - 156) in fp64; the groups of each
//   of S = k >= 1024 ? k / 512 : 1 contiguous slices are added in order from
//   +0 in fp64, the slice sums likewise, and the total is rounded to fp32.
//
// P comes from the matrix core exactly: X_k = sum_d D_d 256^d with signed
// digits D_d in [-128, 127] (the bytes of (X + 0x808080) ^ 0x808080), and
// each MFMA over one group sums digit x code products in int32 (at most
// 128 * 255 * 64 < 2^21 in magnitude), so the hardware's summation order
// cannot change a bit.
//
// MFMA layout (16 x 16 x 64, int8): lane l supplies A row l % 16 and B column
// l % 16 for the 16 k-slots 16 (l / 16) .. +15, and receives D rows
// 4 (l / 16) .. +3 of column l % 16.  A row i = 4 r + d is digit d of
// activation row r of a four-row block (rows 0-3 or 4-7), so lane l ends with
// the four digit sums of activation row l / 16 (+ 4 for the second block)
// against weight row l % 16 of the tile, and combines them in registers.
// Within each lane's 16 k-slots both operands use the k order perm<BITS>():
// 4-bit codes split into low and high nibbles with two masks per word.
#pragma once

#include "common.hpp"

namespace mx {
namespace xq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_a4 __attribute__((ext_vector_type(3), aligned(4)));

constexpr int kGroup = 64;
constexpr int kBlockBytes = 1024;            // A operands of one (group, 4-row block)
constexpr int kGroupBytes = 2 * kBlockBytes; // both blocks of a group
constexpr int kGroupsPerSlice = 8;           // slices of deep rows (k >= 1024)

__host__ __device__ constexpr int slices(int k) { return k >= 1024 ? k / 512 : 1; }

__device__ __forceinline__ v4i mfma(const v4i& a, const v4i& b, const v4i& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Value of the lane's 16 held in operand byte e.
template <int BITS>
__host__ __device__ constexpr int perm(int e) {
  return BITS == 4 ? (e / 8) * 8 + (e % 4) * 2 + (e / 4) % 2 : e;
}

// The lane's code words of one group: 16 codes of value 64 g + 16 kb on.
template <int BITS>
struct Codes {
  static constexpr int W = BITS == 4 ? 2 : BITS == 8 ? 4 : 3;
  uint32_t w[W];
};

// row: the weight row's words; g: group; kb: the lane's 16-value block.
template <int BITS>
__device__ __forceinline__ void load_codes(const uint32_t* __restrict__ row, int g, int kb,
                                           Codes<BITS>& c) {
  if constexpr (BITS == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + 8 * g + 2 * kb);
    c.w[0] = v.x; c.w[1] = v.y;
  } else if constexpr (BITS == 8) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + 16 * g + 4 * kb);
    c.w[0] = v.x; c.w[1] = v.y; c.w[2] = v.z; c.w[3] = v.w;
  } else if constexpr (BITS == 6) {
    const u32x3_a4 v = *reinterpret_cast<const u32x3_a4*>(row + 12 * g + 3 * kb);
    c.w[0] = v.x; c.w[1] = v.y; c.w[2] = v.z;
  } else {  // 5 bits: 80 bits at byte 40 g + 10 kb, a 2-byte aligned offset
    const int byte = 40 * g + 10 * kb;
    const u32x3_a4 v = *reinterpret_cast<const u32x3_a4*>(row + (byte >> 2));
    const uint32_t sh = uint32_t(byte & 3) * 8;
    c.w[0] = __builtin_amdgcn_alignbit(v.y, v.x, sh);
    c.w[1] = __builtin_amdgcn_alignbit(v.z, v.y, sh);
    c.w[2] = v.z >> sh;
  }
}

// 32 bits of the lane's code bits starting at bit B.
template <int BITS, int B>
__device__ __forceinline__ uint32_t bits_at(const Codes<BITS>& c) {
  constexpr int k = B >> 5, o = B & 31;
  if constexpr (o == 0) {
    return c.w[k];
  } else if constexpr (k + 1 < Codes<BITS>::W) {
    return __builtin_amdgcn_alignbit(c.w[k + 1], c.w[k], uint32_t(o));
  } else {
    return c.w[k] >> o;
  }
}

// Four consecutive codes of a window (code i at bit BITS i) as bytes 0..3.
template <int BITS>
__device__ __forceinline__ uint32_t spread4(uint32_t v) {
  constexpr uint32_t m = (1u << BITS) - 1u;
  constexpr int d = 8 - BITS;
  return (v & m) | ((v << d) & (m << 8)) | ((v << (2 * d)) & (m << 16)) |
         ((v << (3 * d)) & (m << 24));
}

// B operand: the lane's 16 codes as int8 in perm<BITS>() order (8-bit codes
// as q - 128, the offset restored through Q in the epilogue).
template <int BITS>
__device__ __forceinline__ v4i b_operand(const Codes<BITS>& c) {
  v4i r;
  if constexpr (BITS == 4) {
    r.x = int(c.w[0] & 0x0F0F0F0Fu);
    r.y = int((c.w[0] >> 4) & 0x0F0F0F0Fu);
    r.z = int(c.w[1] & 0x0F0F0F0Fu);
    r.w = int((c.w[1] >> 4) & 0x0F0F0F0Fu);
  } else if constexpr (BITS == 8) {
    r.x = int(c.w[0] ^ 0x80808080u);
    r.y = int(c.w[1] ^ 0x80808080u);
    r.z = int(c.w[2] ^ 0x80808080u);
    r.w = int(c.w[3] ^ 0x80808080u);
  } else {
    r.x = int(spread4<BITS>(bits_at<BITS, 0>(c)));
    r.y = int(spread4<BITS>(bits_at<BITS, 4 * BITS>(c)));
    r.z = int(spread4<BITS>(bits_at<BITS, 8 * BITS>(c)));
    r.w = int(spread4<BITS>(bits_at<BITS, 12 * BITS>(c)));
  }
  return r;
}

// Grid integer of an fp32-widened bf16 value on the grid 2^(Eb - 156):
// x 2^(156 - Eb) is exact in fp32 (below 2^30) and the conversion truncates
// toward zero.
__device__ __forceinline__ int grid_int(float x, int eb) {
  return int(__builtin_amdgcn_ldexpf(x, 156 - eb));
}

// Signed base-256 digits of X (|X| < 2^30) as the four bytes of a word.
__device__ __forceinline__ uint32_t digits(int X) {
  return (uint32_t(X) + 0x808080u) ^ 0x808080u;
}

// 4 x 4 byte transpose: out[d] byte i = byte d of in[i].
__device__ __forceinline__ void transpose4(const uint32_t (&z)[4], uint32_t (&o)[4]) {
  const uint32_t lo01 = __builtin_amdgcn_perm(z[1], z[0], 0x05010400u);
  const uint32_t hi01 = __builtin_amdgcn_perm(z[1], z[0], 0x07030602u);
  const uint32_t lo23 = __builtin_amdgcn_perm(z[3], z[2], 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(z[3], z[2], 0x07030602u);
  o[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// LDS layout of a staging of `ng` groups: A operands [g][block][lane] x 16 B,
// then Q fp64 [g][8], then Eb int [g][8].
__host__ __device__ constexpr int stage_bytes(int ng) { return ng * (kGroupBytes + 8 * 8 + 8 * 4); }

// Stages groups [g0, g0 + ng) of activation rows xr(0..M-1) (rows past M as
// zeros): the A operands of both four-row blocks in perm<BITS>() order, Q and
// Eb.  All NT threads of the workgroup call it; ends with a barrier.  Each
// wave takes two groups at a time: lane l handles row l % 8 of group
// 2 i + (l % 16) / 8, values 16 (l / 16) .. +15, so the four lanes of one
// (group, row) are 16 apart and share Eb and Q through two butterfly steps.
template <int BITS, int NT, class Rows>
__device__ __forceinline__ void stage(char* lds, const Rows& xr, int M, int g0, int ng) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int NW = NT / 64;
  const int m = lane & 7, kb = lane >> 4, half = (lane >> 3) & 1;
  double* qs = reinterpret_cast<double*>(lds + ng * kGroupBytes);
  int* es = reinterpret_cast<int*>(lds + ng * (kGroupBytes + 64));
  for (int p = wave; 2 * p < ng; p += NW) {
    const int g = 2 * p + half;
    const bool live = g < ng && m < M;
    float f[16];
    if (live) {
      const uint4* src = reinterpret_cast<const uint4*>(xr(m) + size_t(g0 + g) * kGroup + 16 * kb);
      const uint4 a = src[0], b = src[1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        f[2 * i] = u2f(w[i] << 16);
        f[2 * i + 1] = u2f(w[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) f[i] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(f[i]));
    int eb = max(int((f2u(amax) >> 23) & 0xffu), 1);
    eb = max(eb, __shfl_xor(eb, 16, 64));
    eb = max(eb, __shfl_xor(eb, 32, 64));
    int X[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) X[i] = grid_int(f[i], eb);
    double q = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) q += double(X[2 * i] + X[2 * i + 1]);  // pairs < 2^31
    q += __shfl_xor(q, 16, 64);
    q += __shfl_xor(q, 32, 64);
    // operand word p of digit d: bytes i = digit d of value perm(4 p + i)
    uint32_t op[4][4];
#pragma unroll
    for (int pw = 0; pw < 4; ++pw) {
      const uint32_t z[4] = {digits(X[perm<BITS>(4 * pw + 0)]), digits(X[perm<BITS>(4 * pw + 1)]),
                             digits(X[perm<BITS>(4 * pw + 2)]), digits(X[perm<BITS>(4 * pw + 3)])};
      uint32_t t[4];
      transpose4(z, t);
#pragma unroll
      for (int d = 0; d < 4; ++d) op[d][pw] = t[d];
    }
    if (g < ng) {
      char* base = lds + g * kGroupBytes + (m >> 2) * kBlockBytes;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int slot = 4 * (m & 3) + d + 16 * kb;
        *reinterpret_cast<uint4*>(base + slot * 16) = make_uint4(op[d][0], op[d][1], op[d][2], op[d][3]);
      }
      if (kb == 0) {
        qs[g * 8 + m] = q;
        es[g * 8 + m] = eb;
      }
    }
  }
  __syncthreads();
}

// One group of a tile row into the two fp64 row accumulators of this lane
// (activation rows l / 16 and 4 + l / 16 against tile row l % 16): a, Q and
// Eb from the staging (or from registers), s and b the row's scale and bias.
template <int BITS>
__device__ __forceinline__ void group_step(const v4i& a0, const v4i& a1, bool two, const v4i& bop,
                                           double q0, double q1, int e0, int e1, double s,
                                           double b, double (&acc)[2]) {
  const v4i zero = {0, 0, 0, 0};
  const v4i d0 = mfma(a0, bop, zero);
  auto fold = [&](const v4i& d, double q, int e) {
    double p = fma(fma(fma(double(d.w), 256.0, double(d.z)), 256.0, double(d.y)), 256.0,
                   double(d.x));
    if constexpr (BITS == 8) p = p + 128.0 * q;  // codes entered as q - 128
    return __builtin_amdgcn_ldexp(fma(p, s, q * b), e - 156);
  };
  acc[0] = acc[0] + fold(d0, q0, e0);
  if (two) {
    const v4i d1 = mfma(a1, bop, zero);
    acc[1] = acc[1] + fold(d1, q1, e1);
  }
}

}  // namespace xq
}  // namespace mx
