// Matrix-core core of the decode projections for 1..8 activation rows
// (gfx950, v_mfma_f32_16x16x32_bf16), over weights in MLX affine layout.
//
// y[m, n] = sum_g s[n,g] * sum_{k in g} x[m,k] q[n,k] + b[n,g] * sum_{k in g} x[m,k]
// with 64-value groups g.
//
// Work unit of one wave: a tile of 16 weight rows over a range of
// "super-steps" of 128 values (two groups).  Lane l = 16 q + j (j = l % 16,
// q = l / 16) owns weight row j of the tile and, in every super-step, the 32
// consecutive values 32 q .. 32 q + 31 — one 16-byte load at 4 bits, BITS
// dwords in general — which feed four MFMA steps of 8 values each.
//
// MFMA operand layout: lane l supplies A row l % 16 and B column l % 16 for
// the 8 k-slots 8 (l / 16) .. +7, and receives D rows 4 (l / 16) .. +3 of
// column l % 16.  Lane quarter q's k-slots carry values of group 2s + q / 2,
// so one MFMA mixes two groups; they are kept apart through A: row m < 8 holds
// activation m on lanes q < 2 (group 2s) and zero on q >= 2, row m + 8 holds
// activation m on lanes q >= 2 (group 2s + 1) and zero on q < 2.  D rows 0..7
// are then the group-2s sums of the eight activations and rows 8..15 the
// group-(2s+1) sums, and each lane scales its four D values by its own
// group's scale and bias in fp32.  A final exchange between lanes l and
// l + 32 adds the two group parities.  No matrix-core work is wasted for
// M <= 8.
//
// Codes enter the matrix core as exact bf16 integers: for widths <= 7 bits
// (0x4300 | q) is the bf16 value 128 + q, and the 128 * sum(x) this adds is
// removed through the bias (b - 128 s); 8-bit codes are converted exactly
// through fp32.  Within each 8-value unit both operands use the k order
// (0,4,1,5,2,6,3,7), which is how nibble pairs split out of a word.  Products
// are exact; sums are fp32 in the matrix core, then s * acc + b' * sum(x).
//
// The activation rows of a workgroup are staged once in LDS, already in
// operand order: [super-step][u][q][m] x 16 bytes (2 KiB per super-step),
// followed by a 2 KiB zero block that the masked lanes read, and the group
// sums of x as fp32 [group][m].
#pragma once

#include <type_traits>

#include "common.hpp"

namespace mx {
namespace sk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kSuper = 128;       // values per super-step
constexpr int kStepBytes = 2048;  // LDS bytes of staged x per super-step
constexpr int kZeroBytes = 2048;  // zero block read by masked lanes
// Super-steps per weight-load batch: two batches are in flight per wave, so
// a 2048-deep tile of <= 5-bit codes has every load issued up front.
template <int BITS>
constexpr int batch_steps() {
  return BITS <= 5 ? 8 : 4;
}

__device__ __forceinline__ floatx4_t mfma(const uint4& a, const uint4& b, floatx4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Eight bf16 values v0..v7 packed (v0v1, v2v3, v4v5, v6v7) -> operand order
// (v0, v4, v1, v5, v2, v6, v3, v7).
__device__ __forceinline__ uint4 permute_x(const uint4& x) {
  uint4 r;
  r.x = __builtin_amdgcn_perm(x.z, x.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(x.z, x.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(x.w, x.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(x.w, x.y, 0x07060302u);
  return r;
}

template <int BITS>
constexpr float code_offset() {
  return BITS == 8 ? 0.0f : 128.0f;
}

// Four dwords at a dword-aligned address (one 16-byte load; dword-aligned
// vector accesses are legal on gfx950).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// The lane's BITS words of super-step s (values 128 s + 32 q .. +31 of the
// row).  lane: the lane's words of its slice's first super-step (row + 4 BITS
// ks0 + BITS q); s: super-step within the slice (a constant offset once
// unrolled).
template <int BITS>
__device__ __forceinline__ void load_codes(const uint32_t* __restrict__ lane, int s,
                                           uint32_t (&w)[BITS]) {
  const uint32_t* p = lane + (4 * BITS) * s;
  if constexpr (BITS == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (BITS == 8) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (BITS == 6) {
    // 24 bytes at an 8-byte aligned offset: a 16-byte and an 8-byte load
    const u32x4_a4 a = *reinterpret_cast<const u32x4_a4*>(p);
    const uint2 b = *reinterpret_cast<const uint2*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y;
  } else if constexpr (BITS == 5) {
    // 20 bytes at a 4-byte aligned offset: a 16-byte load and a dword
    const u32x4_a4 a = *reinterpret_cast<const u32x4_a4*>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = p[4];
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = p[i];
  }
}

// Value V (0..31) of the lane's words.
template <int BITS, int V>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&w)[BITS]) {
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

// 0x43004300 in a vector register: with the mask in a scalar register,
// (p & mask) | c is then one v_and_or_b32 (a VOP3 instruction takes neither
// literal operands nor two scalar registers on this architecture).
__device__ __forceinline__ uint32_t vconst_43004300() {
  uint32_t c;
  asm("v_mov_b32 %0, 0x43004300" : "=v"(c));
  return c;
}

// The 32 bits of the lane's words starting at bit BIT (bits past the last
// word read as zeros).
template <int BITS, int BIT>
__device__ __forceinline__ uint32_t window(const uint32_t (&w)[BITS]) {
  constexpr int k = BIT >> 5, o = BIT & 31;
  if constexpr (o == 0) {
    return w[k];
  } else if constexpr (k + 1 < BITS) {
    return __builtin_amdgcn_alignbit(w[k + 1], w[k], uint32_t(o));
  } else {
    return w[k] >> o;
  }
}

// B operand of MFMA step U (values 8U .. 8U+7 of the lane's 32) in operand order.
template <int BITS, int U>
__device__ __forceinline__ uint4 b_operand(const uint32_t (&w)[BITS]) {
  uint4 r;
  if constexpr (BITS == 4) {
    // nibbles as bytes (lo: n0 n2 n4 n6, hi: n1 n3 n5 n7), then one byte
    // permute per operand word places two of them under 0x43 high bytes
    const uint32_t x = w[U];
    const uint32_t lo = x & 0x0F0F0F0Fu;
    const uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;
    constexpr uint32_t c43 = 0x43434343u;
    r.x = __builtin_amdgcn_perm(lo, c43, 0x00060004u);  // n0, n4
    r.y = __builtin_amdgcn_perm(hi, c43, 0x00060004u);  // n1, n5
    r.z = __builtin_amdgcn_perm(lo, c43, 0x00070005u);  // n2, n6
    r.w = __builtin_amdgcn_perm(hi, c43, 0x00070005u);  // n3, n7
  } else if constexpr (BITS == 8) {
    const uint32_t lo = w[2 * U], hi = w[2 * U + 1];
    auto pair = [](float a, float b) { return __builtin_amdgcn_perm(f2u(b), f2u(a), 0x07060302u); };
    r.x = pair(float(lo & 0xffu), float(hi & 0xffu));
    r.y = pair(float((lo >> 8) & 0xffu), float((hi >> 8) & 0xffu));
    r.z = pair(float((lo >> 16) & 0xffu), float((hi >> 16) & 0xffu));
    r.w = pair(float(lo >> 24), float(hi >> 24));
  } else if constexpr (BITS == 5) {
    // the operand's codes are the 40 bits at b = 40 U and each operand word
    // pairs codes i and i + 4, 20 bits apart: one word p holding bits
    // b .. b+15 low and b+20 .. b+35 high yields pairs 0..2 as
    // (p >> 5 i) & 0x001F001F; pair 3 comes from windows at b+15 and b+19
    constexpr int b = 40 * U;
    constexpr uint32_t m = 0x001F001Fu;
    const uint32_t c = vconst_43004300();
    const uint32_t p = (window<5, b>(w) & 0xFFFFu) | (window<5, b + 4>(w) & 0xFFFF0000u);
    const uint32_t p3 = (window<5, b + 15>(w) & 0xFFFFu) | (window<5, b + 19>(w) & 0xFFFF0000u);
    r.x = (p & m) | c;
    r.y = ((p >> 5) & m) | c;
    r.z = ((p >> 10) & m) | c;
    r.w = (p3 & m) | c;
  } else if constexpr (BITS == 6) {
    // 48 bits at b = 48 U, pairs 24 bits apart: words holding bits b .. +15
    // with b+24 .. +39 (pairs 0, 1) and b+12 .. +27 with b+36 .. +51 (2, 3)
    constexpr int b = 48 * U;
    constexpr uint32_t m = 0x003F003Fu;
    const uint32_t c = vconst_43004300();
    const uint32_t p = (window<6, b>(w) & 0xFFFFu) | (window<6, b + 8>(w) & 0xFFFF0000u);
    const uint32_t p2 = (window<6, b + 12>(w) & 0xFFFFu) | (window<6, b + 20>(w) & 0xFFFF0000u);
    r.x = (p & m) | c;
    r.y = ((p >> 6) & m) | c;
    r.z = (p2 & m) | c;
    r.w = ((p2 >> 6) & m) | c;
  } else {
    r.x = (code_at<BITS, 8 * U + 0>(w) | (code_at<BITS, 8 * U + 4>(w) << 16)) | 0x43004300u;
    r.y = (code_at<BITS, 8 * U + 1>(w) | (code_at<BITS, 8 * U + 5>(w) << 16)) | 0x43004300u;
    r.z = (code_at<BITS, 8 * U + 2>(w) | (code_at<BITS, 8 * U + 6>(w) << 16)) | 0x43004300u;
    r.w = (code_at<BITS, 8 * U + 3>(w) | (code_at<BITS, 8 * U + 7>(w) << 16)) | 0x43004300u;
  }
  return r;
}

// Stages activation rows xr(0..7) (nullptr = zero row) for super-steps
// [ks0, ks0 + steps) of a K-long row into LDS, with the zero block and the
// per-group sums of x.  Called by all 256 threads; ends with a barrier.
// Activation rows of a plain projection: row m at x + m * stride, m < M.
struct DenseRows {
  const uint16_t* x;
  int64_t stride;
  int M;
  __device__ __forceinline__ const uint16_t* operator()(int m) const {
    return m < M ? x + m * stride : nullptr;
  }
};

// Activation rows of an expert chunk: member m (< M) is route (row, slot)
// packed as 8 bits (row << 5 | slot) at bit 8 m of `packed`; its row lies at
// base + row * row_stride + slot * slot_stride.
struct RouteRows {
  const uint16_t* base;
  int64_t row_stride, slot_stride;
  uint64_t packed;
  int M;
  __device__ __forceinline__ int row(int m) const { return int((packed >> (8 * m)) & 0xffu) >> 5; }
  __device__ __forceinline__ int slot(int m) const { return int((packed >> (8 * m)) & 0x1fu); }
  __device__ __forceinline__ const uint16_t* operator()(int m) const {
    return m < M ? base + row(m) * row_stride + slot(m) * slot_stride : nullptr;
  }
};

// Stages, for the workgroup's super-steps [ks0, ks0 + steps) of K-long rows:
// the x tile in operand order, the zero block and the group sums of x (fp32
// [group][m] after the zero block).  Rows past the first M stage as zeros.
// Unit i (16 bytes) of the staging is value unit u = i / 8 of row m = i % 8,
// so the 64 lanes of a wave hold the eight units of one 64-value group for
// all eight rows: their LDS stores spread over the banks (consecutive lanes
// write different rows), and each group's sum is a butterfly over lanes 8
// apart.  load() issues every global load of the staging (unconditionally:
// rows past M load row M - 1, whose address the wave already touches);
// store() waits for them, writes LDS and ends with a barrier.  Loads issued
// between the two (the weight prefetch) stay in flight, because the hardware
// retires loads in order and store() only needs the older ones.  One pass
// covers NT * PER 16-byte units; the staging must fit one pass.
template <int NT, int PER, class Rows>
struct Stager {
  const Rows& xr;
  int live, ks0, steps, total;
  uint4 v[PER];

  // M: rows xr(0..M-1) exist (the others stage as zeros and are not loaded).
  __device__ __forceinline__ Stager(const Rows& r, int M, int k0, int n)
      : xr(r), live(M), ks0(k0), steps(n), total(8 * n * 16) {}

  __device__ __forceinline__ void load() {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int i = min(int(threadIdx.x) + k * NT, total - 1);
      const int m = min(i & 7, live - 1), u = i >> 3;
      v[k] = *reinterpret_cast<const uint4*>(xr(m) + size_t(ks0) * kSuper + u * 8);
    }
  }

  __device__ __forceinline__ void store(char* lds) {
    const int xbytes = steps * kStepBytes;
    uint4* xs = reinterpret_cast<uint4*>(lds);
    float* sx = reinterpret_cast<float*>(lds + xbytes + kZeroBytes);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      if (k * NT >= total) break;  // uniform
      const int i = int(threadIdx.x) + k * NT;
      if (i - int(threadIdx.x & 63) >= total) break;  // uniform per wave (total % 64 == 0)
      const int m = i & 7, u = i >> 3;
      const uint4 val = m < live ? v[k] : make_uint4(0, 0, 0, 0);
      const uint32_t d[4] = {val.x, val.y, val.z, val.w};
      float sum = 0.0f;
#pragma unroll
      for (int h = 0; h < 4; ++h) sum = sum + u2f(d[h] << 16) + u2f(d[h] & 0xffff0000u);
      sum = sum + __shfl_xor(sum, 8, 64);
      sum = sum + __shfl_xor(sum, 16, 64);
      sum = sum + __shfl_xor(sum, 32, 64);
      if ((u & 7) == 0) sx[(u >> 3) * 8 + m] = sum;
      const int s = u >> 4, o = u & 15;
      xs[(s * 4 + (o & 3)) * 32 + (o >> 2) * 8 + m] = permute_x(val);
    }
    uint2* zero = reinterpret_cast<uint2*>(lds + xbytes);
    for (int t = threadIdx.x; t < kZeroBytes / 8; t += NT) zero[t] = make_uint2(0, 0);
    __syncthreads();
  }
};

// Units per thread that stage `steps` super-steps in one pass with NT threads.
__host__ __device__ constexpr int stage_per(int nt, int steps) {
  return (8 * 16 * steps + nt - 1) / nt;
}

// LDS bytes of a staging for `steps` super-steps.
__host__ __device__ constexpr int stage_bytes(int steps) {
  return steps * kStepBytes + kZeroBytes + steps * 2 * 8 * 4;
}

// One wave's stream over a tile row: super-steps [ks0, ks0 + steps) of the
// row `crow` (scales `srow`, biases `brow`), accumulated into y[4] (this
// lane's D rows, before the parity exchange).  The activations come from the
// staged x tile (XREG = false; super-step ks at local index ks - wks0, group
// sums staged too) or, XREG = true, straight from the rows xr(m) into
// registers, with the group sums from one more MFMA against ones.
//
// Scales and biases: lane quarter q loads, with one SCW-byte load each, the
// words of super-steps base + SQ q .. base + SQ q + SQ - 1 (SQ = SCW / 4; a
// word holds the two groups of a super-step), base = ks0 rounded down to SQ;
// each super-step takes its word from the owning quarter with a lane shuffle.
// The slice must satisfy (ks0 % SQ) + steps <= 4 SQ and, for SCW = 16, a row's
// scales must start 16-byte aligned (K % 512 == 0).
// prefetch() issues the scale words and the first two batches; run() does
// the rest.  Loads are unconditional (indices past the slice are clamped to
// its last super-step): no branch separates them, so the compiler's wait
// counts stay exact and later batches stay in flight.
template <int BITS, bool XREG, class Rows, int BMAX = 8, int SCW = 16>
struct Stream {
  static constexpr int B =
      XREG ? 1 : (batch_steps<BITS>() < BMAX ? batch_steps<BITS>() : BMAX);
  static constexpr int SQ = SCW / 4;
  typedef typename std::conditional<SCW == 16, uint4, uint2>::type Quad;
  const uint32_t* cq;     // the lane's words of the slice's first super-step
  const uint16_t* srow;
  const uint16_t* brow;
  int ks0, steps, wks0, base, row_steps;
  const char* lds;   // staged x tile (XREG = false)
  const float* sx;   // staged group sums (XREG = false)
  const uint16_t* xrow;  // the lane's activations of the slice's first super-step (XREG = true)
  bool xlive;            // the lane's A operand is live (XREG = true)
  Quad scq, bcq;
  uint32_t wa[B][BITS], wb[B][BITS];
  uint4 xa[XREG ? B : 1][4], xb[XREG ? B : 1][4];
  int j, q, xoff, zoff;
  uint32_t half_sel;  // byte permute that moves this lane's group half to the top
  bool act;

  // rs: super-steps in the whole row (K / 128, a multiple of SQ).
  __device__ __forceinline__ Stream(const uint32_t* c, const uint16_t* sr, const uint16_t* br,
                                    int rs, int k0, int n, int w0, const char* l, const float* s,
                                    const Rows& xr, int M)
      : srow(sr), brow(br), ks0(k0), steps(n), wks0(w0), row_steps(rs), lds(l), sx(s) {
    const int lane = threadIdx.x & 63;
    j = lane & 15;
    q = lane >> 4;
    cq = c + size_t(4 * BITS) * ks0 + BITS * q;
    base = ks0 - ks0 % SQ;
    half_sel = (q >> 1) ? 0x07060c0cu : 0x05040c0cu;
    act = (j < 8) == (q < 2);
    xoff = (q * 8 + (j & 7)) * 16;
    xlive = false;
    xrow = nullptr;
    if constexpr (XREG) {
      xlive = act && (j & 7) < M;
      xrow = xr((j & 7) < M ? (j & 7) : 0) + size_t(ks0) * kSuper + 32 * q;
    }
  }

  __device__ __forceinline__ void load(uint32_t (&w)[B][BITS], uint4 (&xv)[XREG ? B : 1][4],
                                       int s0) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      // super-steps past the slice are clamped to its last one
      const int ls = min(s0 + i, steps - 1);
      load_codes<BITS>(cq, ls, w[i]);
      if constexpr (XREG) {
        const uint4* p = reinterpret_cast<const uint4*>(xrow + ls * kSuper);
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[i][u] = p[u];
      }
    }
  }

  __device__ __forceinline__ static uint32_t word(const Quad& v, int i) {
    if constexpr (SCW == 16) {
      return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
    } else {
      return i == 0 ? v.x : v.y;
    }
  }

  __device__ __forceinline__ void compute(const uint32_t (&w)[B][BITS],
                                          const uint4 (&xv)[XREG ? B : 1][4], int s0,
                                          float (&y)[4]) {
    const float off = code_offset<BITS>();
    const int hi = q >> 1;
    const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int s = s0 + i;
      if (s < steps) {
        const int rel = ks0 + s - base;
        const int src = j + 16 * (rel / SQ);
        const uint32_t sw = uint32_t(__shfl(int(word(scq, rel % SQ)), src, 64));
        const uint32_t bw = uint32_t(__shfl(int(word(bcq, rel % SQ)), src, 64));
        uint4 a[4];
        floatx4_t sv;
        if constexpr (XREG) {
#pragma unroll
          for (int u = 0; u < 4; ++u)
            a[u] = xlive ? permute_x(xv[i][u]) : make_uint4(0, 0, 0, 0);
          floatx4_t sa = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int u = 0; u < 4; ++u) sa = mfma(a[u], ones, sa);
          sv = sa;
        } else {
          const int ls = ks0 + s - wks0;  // local super-step of the staging
          const char* ap = lds + (act ? ls * kStepBytes + xoff : zoff);
#pragma unroll
          for (int u = 0; u < 4; ++u) a[u] = *reinterpret_cast<const uint4*>(ap + 512 * u);
          sv = *reinterpret_cast<const floatx4_t*>(sx + (2 * ls + hi) * 8 + 4 * (q & 1));
        }
        floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = mfma(a[0], b_operand<BITS, 0>(w[i]), acc);
        acc = mfma(a[1], b_operand<BITS, 1>(w[i]), acc);
        acc = mfma(a[2], b_operand<BITS, 2>(w[i]), acc);
        acc = mfma(a[3], b_operand<BITS, 3>(w[i]), acc);
        const float sc = u2f(__builtin_amdgcn_perm(sw, sw, half_sel));
        const float bi = fmaf_(-off, sc, u2f(__builtin_amdgcn_perm(bw, bw, half_sel)));
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = fmaf_(sc, acc[r], fmaf_(bi, sv[r], y[r]));
      }
    }
  }

  // Issues the scale words and the first two batches.
  __device__ __forceinline__ void prefetch() {
    const int qs = min(base + SQ * q, row_steps - SQ);
    scq = *reinterpret_cast<const Quad*>(srow + 2 * qs);
    bcq = *reinterpret_cast<const Quad*>(brow + 2 * qs);
    load(wa, xa, 0);
    if (B < steps) load(wb, xb, B);
  }

  // zero_off: byte offset of the zero block in the staged tile (XREG = false).
  __device__ __forceinline__ void run(int zero_off, float (&y)[4]) {
    zoff = zero_off;
    if (steps <= 2 * B) {
      // both batches are already in flight: straight-line code keeps the
      // compiler's wait counts exact (no loop-header merge)
      compute(wa, xa, 0, y);
      if (B < steps) compute(wb, xb, B, y);
      return;
    }
    for (int s0 = 0; s0 < steps; s0 += 2 * B) {
      compute(wa, xa, s0, y);
      if (s0 + 2 * B < steps) load(wa, xa, s0 + 2 * B);
      if (s0 + B < steps) {
        compute(wb, xb, s0 + B, y);
        if (s0 + 3 * B < steps) load(wb, xb, s0 + 3 * B);
      }
    }
  }
};

// Adds the two group parities: lanes q < 2 end with the sums of activations
// 4 q + r (r < 4) for tile row j.
__device__ __forceinline__ void join_parities(float (&y)[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = y[r] + __shfl_xor(y[r], 32, 64);
}

}  // namespace sk
}  // namespace mx
