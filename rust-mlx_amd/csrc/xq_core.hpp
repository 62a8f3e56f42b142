// Exact-integer projection core for 1..8 activation rows (gfx950,
// v_mfma_i32_16x16x64_i8), over weights in MLX's affine layout.
//
// The arithmetic (restated by the CPU oracle, oracle/xq.c):
//   per 64-value group g of activation row m, Eb = the largest bf16 exponent
//   field of the group (at least 1) and X_k = trunc(x_k 2^(156 - Eb)), an
//   integer below 2^30 in magnitude; P = sum X_k q_k and Q = sum X_k are
//   exact; v_g = fma(P, s_g, Q b_g) 2^(Eb - 156) in fp64; the groups of each
//   slice of two consecutive groups are added in order from +0 in fp64, the
//   slice sums likewise, and the total is rounded to fp32.
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
// Within each lane's 16 k-slots both operands use one k order, perm(): the
// order in which 4-bit codes split into low and high nibbles with two masks
// per word (other widths are permuted into it), so an activation plane built
// once serves every consumer whatever its code width.
#pragma once

#include "common.hpp"

namespace mx {
namespace xq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_a4 __attribute__((ext_vector_type(3), aligned(4)));

constexpr int kGroup = 64;
constexpr int kBlockBytes = 1024;            // A operands of one (group, 4-row block)
constexpr int kGroupBytes = 2 * kBlockBytes; // both blocks of a group

// Slices of the arithmetic: two consecutive groups each (the last of an odd
// count holds one).
__host__ __device__ constexpr int slices(int k) { return (k / kGroup + 1) / 2; }

__device__ __forceinline__ v4i mfma(const v4i& a, const v4i& b, const v4i& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Value of the lane's 16 held in operand byte e: bytes 0-3 hold values
// 0, 2, 4, 6; 4-7 values 1, 3, 5, 7; 8-11 values 8 .. 14; 12-15 values 9 .. 15.
__host__ __device__ constexpr int perm(int e) { return (e / 8) * 8 + (e % 4) * 2 + (e / 4) % 2; }

// Words of values (0..3, 4..7) -> (0, 2, 4, 6) and (1, 3, 5, 7).
__device__ __forceinline__ int even_of(uint32_t lo, uint32_t hi) {
  return int(__builtin_amdgcn_perm(hi, lo, 0x06040200u));
}
__device__ __forceinline__ int odd_of(uint32_t lo, uint32_t hi) {
  return int(__builtin_amdgcn_perm(hi, lo, 0x07050301u));
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

// B operand: the lane's 16 codes as int8 in perm() order (8-bit codes as
// q - 128, the offset restored through Q in the epilogue).
template <int BITS>
__device__ __forceinline__ v4i b_operand(const Codes<BITS>& c) {
  v4i r;
  if constexpr (BITS == 4) {
    r.x = int(c.w[0] & 0x0F0F0F0Fu);
    r.y = int((c.w[0] >> 4) & 0x0F0F0F0Fu);
    r.z = int(c.w[1] & 0x0F0F0F0Fu);
    r.w = int((c.w[1] >> 4) & 0x0F0F0F0Fu);
  } else if constexpr (BITS == 8) {
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = c.w[i] ^ 0x80808080u;
    r.x = even_of(q[0], q[1]);
    r.y = odd_of(q[0], q[1]);
    r.z = even_of(q[2], q[3]);
    r.w = odd_of(q[2], q[3]);
  } else {
    // 5 / 6 bits: each code extracted from a 32-bit window holding it whole
    // (w0 = bits 0..31, then bits 30..61 and 60..91 of the lane's codes) and
    // shifted into its byte: the same bytes as spreading four codes at a
    // time and interleaving them, in fewer instructions
    const uint32_t wa = c.w[0];
    const uint32_t wb = __builtin_amdgcn_alignbit(c.w[1], c.w[0], 30u);
    const uint32_t wc = __builtin_amdgcn_alignbit(c.w[2], c.w[1], 28u);
    auto code = [&](int i) -> uint32_t {
      const int at = BITS * i;  // compile-time after unrolling
      const uint32_t src = at + BITS <= 32 ? wa : at + BITS <= 62 ? wb : at + BITS <= 92 ? wc : c.w[2];
      const int off = at + BITS <= 32 ? at : at + BITS <= 62 ? at - 30 : at + BITS <= 92 ? at - 60 : at - 64;
      return __builtin_amdgcn_ubfe(src, uint32_t(off), uint32_t(BITS));
    };
    auto pack = [&](int a) -> int {  // codes a, a + 2, a + 4, a + 6 as bytes 0..3
      return int(code(a) | (code(a + 2) << 8) | (code(a + 4) << 16) | (code(a + 6) << 24));
    };
    r.x = pack(0);
    r.y = pack(1);
    r.z = pack(8);
    r.w = pack(9);
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

// Layout of the activation operands of `ng` groups, in LDS (a staging) or in
// global memory (a plane written by the producer of the activations):
// A operands [g][block][lane] x 16 B, then Q fp64 [g][8], then Eb int [g][8].
__host__ __device__ constexpr int stage_bytes(int ng) { return ng * (kGroupBytes + 8 * 8 + 8 * 4); }
__host__ __device__ constexpr int plane_q_offset(int ng) { return ng * kGroupBytes; }
__host__ __device__ constexpr int plane_e_offset(int ng) { return ng * (kGroupBytes + 64); }

// One 16-value unit of activation row m (< 8), values 16 kb .. +15 of group
// g: f holds them widened to fp32.  The four lanes holding one (group, row)
// must be 16 apart in the wave (kb = lane / 16): they share Eb and Q through
// two butterfly steps.  Writes the unit's four digit operands, and (kb == 0)
// Q and Eb, into the layout of `ng` groups at dst; `write` false still joins
// the butterflies.
__device__ __forceinline__ void digitize_unit(const float (&f)[16], int m, int g, int kb,
                                              bool write, char* dst, int ng) {
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
  if (!write) return;
  // operand word p of digit d: byte i = digit d of value perm(4 p + i)
  uint32_t op[4][4];
#pragma unroll
  for (int pw = 0; pw < 4; ++pw) {
    const uint32_t z[4] = {digits(X[perm(4 * pw + 0)]), digits(X[perm(4 * pw + 1)]),
                           digits(X[perm(4 * pw + 2)]), digits(X[perm(4 * pw + 3)])};
    uint32_t t[4];
    transpose4(z, t);
#pragma unroll
    for (int d = 0; d < 4; ++d) op[d][pw] = t[d];
  }
  char* base = dst + g * kGroupBytes + (m >> 2) * kBlockBytes;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int slot = 4 * (m & 3) + d + 16 * kb;
    *reinterpret_cast<uint4*>(base + slot * 16) = make_uint4(op[d][0], op[d][1], op[d][2], op[d][3]);
  }
  if (kb == 0) {
    reinterpret_cast<double*>(dst + plane_q_offset(ng))[g * 8 + m] = q;
    reinterpret_cast<int*>(dst + plane_e_offset(ng))[g * 8 + m] = eb;
  }
}

// Widens 16 bf16 values (two 16-byte loads) to fp32.
__device__ __forceinline__ void load16(const uint16_t* src, float (&f)[16]) {
  const uint4 a = reinterpret_cast<const uint4*>(src)[0], b = reinterpret_cast<const uint4*>(src)[1];
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f[2 * i] = u2f(w[i] << 16);
    f[2 * i + 1] = u2f(w[i] & 0xffff0000u);
  }
}

// Stages groups [g0, g0 + ng) of activation rows xr(0..M-1) into LDS.  Rows
// past M are left unwritten: their matrix-core sums land in D rows that no
// epilogue reads.  All NT threads of the workgroup call it; ends with a
// barrier.  Each wave takes 16 / R groups at a time (R = 8 rows rounded up to
// a power of two >= M): lane l handles row (l % 16) % R of group
// i + (l % 16) / R, values 16 (l / 16) .. +15.
template <int NT, class Rows>
__device__ __forceinline__ void stage(char* lds, const Rows& xr, int M, int g0, int ng) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int NW = NT / 64;
  const int R = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const int per = 16 / R;  // groups per wave step
  const int m = (lane & 15) % R, kb = lane >> 4, sub = (lane & 15) / R;
  for (int p = wave; p * per < ng; p += NW) {
    const int g = p * per + sub;
    const bool live = g < ng && m < M;
    float f[16];
    if (live) {
      load16(xr(m) + size_t(g0 + g) * kGroup + 16 * kb, f);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) f[i] = 0.0f;
    }
    digitize_unit(f, m, g, kb, live, lds, ng);
  }
  __syncthreads();
}

// Copies an activation plane of G groups (the layout above) into LDS with
// direct global-to-LDS loads, 16 bytes per lane, no registers held; all NT
// threads of the workgroup call it.  Ends with every load landed and a
// barrier.
template <int NT>
__device__ __forceinline__ void dma_plane(char* lds, const char* __restrict__ plane, int G) {
  const int n16 = stage_bytes(G) / 16;
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < n16; i += NT) {
    // the wave's lanes land at consecutive 16-byte slots from its first index
    __builtin_amdgcn_global_load_lds(
        plane + size_t(i) * 16,
        reinterpret_cast<__attribute__((address_space(3))) void*>(
            reinterpret_cast<uintptr_t>(lds + size_t(i - lane) * 16)),
        16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// One four-row block of an activation plane in LDS: the A operands of block
// `blk` of every group (1 KB a group), then Q [g][8], then Eb [g][8] of all
// eight rows, copied like dma_plane.
__host__ __device__ constexpr int block_bytes(int ng) { return ng * (kBlockBytes + 8 * 8 + 8 * 4); }
__host__ __device__ constexpr int block_q_offset(int ng) { return ng * kBlockBytes; }
__host__ __device__ constexpr int block_e_offset(int ng) { return ng * (kBlockBytes + 64); }

// `rot` (any value) rotates the order of the 1 KB pieces: workgroups that
// copy the same plane at once start at different places, so their requests
// spread over the cache channels instead of queueing on the same lines.
template <int NT>
__device__ __forceinline__ void dma_plane_block(char* lds, const char* __restrict__ plane, int G,
                                                int blk, int rot = 0) {
  const int na = G * (kBlockBytes / 16), n16 = block_bytes(G) / 16;
  const int pieces = (n16 + 63) / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  rot = rot % pieces;
  for (int p = wave; p < pieces; p += NT / 64) {
    int q = p + rot;
    q = q >= pieces ? q - pieces : q;  // this instruction's 1 KB piece
    const int i = q * 64 + lane;
    if (i < n16) {
      const char* src = i < na ? plane + size_t(i >> 6) * kGroupBytes + blk * kBlockBytes +
                                     (i & 63) * 16
                               : plane + plane_q_offset(G) + size_t(i - na) * 16;
      __builtin_amdgcn_global_load_lds(
          src,
          reinterpret_cast<__attribute__((address_space(3))) void*>(
              reinterpret_cast<uintptr_t>(lds + size_t(q) * 1024)),
          16, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Scales and biases of B consecutive groups of one weight row, as bf16 pairs.
template <int B>
struct ScaleBias {
  static constexpr int W = (B + 1) / 2;
  uint32_t s[W], b[W];
  __device__ __forceinline__ double scale(int i) const { return half(s[i >> 1], i); }
  __device__ __forceinline__ double bias(int i) const { return half(b[i >> 1], i); }
  __device__ __forceinline__ static double half(uint32_t w, int i) {
    return double(u2f((i & 1) ? (w & 0xffff0000u) : (w << 16)));
  }
};

// Whether the scale and bias rows of a matrix with G groups per row can be
// read B values at a time: G a multiple of B and both arrays starting on a
// 2B-byte boundary (then every row and every batch start on one too).
template <int B>
__host__ __device__ __forceinline__ bool sb_vector_ok(const uint16_t* scales,
                                                      const uint16_t* biases, int G) {
  const uintptr_t at = reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases);
  return B > 1 && G % B == 0 && (at & uintptr_t(2 * B - 1)) == 0;
}

// Groups g0 .. g0 + B - 1 of the row's scales and biases with one vector load
// each: the caller guarantees g0 % B == 0, g0 + B <= G and sb_vector_ok.
template <int B>
__device__ __forceinline__ void load_scale_bias_vec(const uint16_t* __restrict__ srow,
                                                    const uint16_t* __restrict__ brow, int g0,
                                                    ScaleBias<B>& o) {
  static_assert(B == 2 || B == 4 || B == 8, "batch");
  if constexpr (B == 8) {
    const uint4 sv = *reinterpret_cast<const uint4*>(srow + g0);
    const uint4 bv = *reinterpret_cast<const uint4*>(brow + g0);
    o.s[0] = sv.x; o.s[1] = sv.y; o.s[2] = sv.z; o.s[3] = sv.w;
    o.b[0] = bv.x; o.b[1] = bv.y; o.b[2] = bv.z; o.b[3] = bv.w;
  } else if constexpr (B == 4) {
    const uint2 sv = *reinterpret_cast<const uint2*>(srow + g0);
    const uint2 bv = *reinterpret_cast<const uint2*>(brow + g0);
    o.s[0] = sv.x; o.s[1] = sv.y;
    o.b[0] = bv.x; o.b[1] = bv.y;
  } else {
    o.s[0] = *reinterpret_cast<const uint32_t*>(srow + g0);
    o.b[0] = *reinterpret_cast<const uint32_t*>(brow + g0);
  }
}

// Groups g0 .. g0 + B - 1 of the row's scales and biases, indices clamped to
// gend - 1: one vector load each when `vec` (sb_vector_ok of the matrix) and
// the batch starts on a multiple of B and lies below gend.  Every argument
// but the row pointers is the same across the wave, so the choice is too.
template <int B>
__device__ __forceinline__ void load_scale_bias(const uint16_t* __restrict__ srow,
                                                const uint16_t* __restrict__ brow, int g0,
                                                int gend, bool vec, ScaleBias<B>& o) {
  static_assert(B == 1 || B == 2 || B == 4 || B == 8, "batch");
  if (B > 1 && vec && g0 % B == 0 && g0 + B <= gend) {
    if constexpr (B == 8) {
      const uint4 sv = *reinterpret_cast<const uint4*>(srow + g0);
      const uint4 bv = *reinterpret_cast<const uint4*>(brow + g0);
      o.s[0] = sv.x; o.s[1] = sv.y; o.s[2] = sv.z; o.s[3] = sv.w;
      o.b[0] = bv.x; o.b[1] = bv.y; o.b[2] = bv.z; o.b[3] = bv.w;
    } else if constexpr (B == 4) {
      const uint2 sv = *reinterpret_cast<const uint2*>(srow + g0);
      const uint2 bv = *reinterpret_cast<const uint2*>(brow + g0);
      o.s[0] = sv.x; o.s[1] = sv.y;
      o.b[0] = bv.x; o.b[1] = bv.y;
    } else if constexpr (B == 2) {
      o.s[0] = *reinterpret_cast<const uint32_t*>(srow + g0);
      o.b[0] = *reinterpret_cast<const uint32_t*>(brow + g0);
    }
  } else {
#pragma unroll
    for (int w = 0; w < ScaleBias<B>::W; ++w) {
      const int ga = min(g0 + 2 * w, gend - 1), gb = min(g0 + 2 * w + 1, gend - 1);
      o.s[w] = uint32_t(srow[ga]) | (uint32_t(srow[gb]) << 16);
      o.b[w] = uint32_t(brow[ga]) | (uint32_t(brow[gb]) << 16);
    }
  }
}

// One group of a tile row into the two fp64 row accumulators of this lane
// (activation rows l / 16 and 4 + l / 16 against tile row l % 16) for the
// four-row blocks in `blocks` (bit 0: rows 0-3, bit 1: rows 4-7): a, Q and Eb
// of each block's row, s and b the tile row's scale and bias.
template <int BITS, int BLK>
__device__ __forceinline__ void group_step(const v4i& a0, const v4i& a1, const v4i& bop,
                                           double q0, double q1, int e0, int e1, double s,
                                           double b, double (&acc)[2]) {
  const v4i zero = {0, 0, 0, 0};
  auto fold = [&](const v4i& d, double q, int e) {
    // P = (D0 + 256 D1) + 65536 (D2 + 256 D3): each pair is exact in int32
    // (|D| < 2^21) and the fp64 combination is exact (|P| < 2^47)
    const int lo = d.x + d.y * 256, hi = d.z + d.w * 256;
    double p = fma(double(hi), 65536.0, double(lo));
    if constexpr (BITS == 8) p = fma(q, 128.0, p);  // codes entered as q - 128
    return __builtin_amdgcn_ldexp(fma(p, s, q * b), e - 156);
  };
  if constexpr (BLK & 1) acc[0] = acc[0] + fold(mfma(a0, bop, zero), q0, e0);
  if constexpr (BLK & 2) acc[1] = acc[1] + fold(mfma(a1, bop, zero), q1, e1);
}

// One group of one four-row block: a, Q and Eb of the lane's activation row
// of that block, s and b the tile row's scale and bias.
template <int BITS>
__device__ __forceinline__ void group_step1(const v4i& a, const v4i& bop, double q, int e,
                                            double s, double b, double& acc) {
  double pair[2] = {acc, 0.0};
  group_step<BITS, 1>(a, a, bop, q, q, e, e, s, b, pair);
  acc = pair[0];
}

// The same with the blocks chosen at run time (uniform across the wave).
template <int BITS>
__device__ __forceinline__ void group_step(const v4i& a0, const v4i& a1, int blocks,
                                           const v4i& bop, double q0, double q1, int e0, int e1,
                                           double s, double b, double (&acc)[2]) {
  if (blocks & 1) group_step<BITS, 1>(a0, a1, bop, q0, q1, e0, e1, s, b, acc);
  if (blocks & 2) group_step<BITS, 2>(a0, a1, bop, q0, q1, e0, e1, s, b, acc);
}

}  // namespace xq
}  // namespace mx
