// Affine-quantised matvec / skinny GEMM for 1..8 activation rows (gfx950).
//
// Replaces reference kernels/verify_qmv.{h,metal} (dispatched from
// src/qmv_kernel.rs:49-180) and the native quantized_matmul / gather_qmm rows
// of Linear::forward_rows (src/weights.rs:111-202).
//
// Arithmetic contract (the fixed order a CPU restatement reproduces bit for
// bit).  For output row n and activation row m:
//   * the K axis is cut into 32-value chunks c = 0 .. K/32-1;
//   * acc_c = fma chain over j = 0..31 of x[32c+j] * q[32c+j], starting at 0;
//   * sx_c  = sequential fp32 sum of x[32c+j], j = 0..31;
//   * part_c = fma(scale_g, acc_c, bias_g * sx_c), g = 32c / group_size
//     (MLX's  s * sum(x q) + b * sum(x)  form, reference verify_qmv.h:112);
//   * L = min(64, largest power of two <= K/32) lanes share a row; lane l
//     sums part_c for c = l, l+L, l+2L, ... in ascending order from +0;
//   * an xor butterfly over the L lanes (offsets L/2, ..., 1) adds the lane
//     sums; the result is rounded to bf16 (round to nearest even).
// The order depends on K only, never on the number of activation rows, so a
// batch of rows gives the same bits as each row alone.
#include "common.hpp"
#include "kernels.hpp"

namespace mx {

namespace {

constexpr int kRowsPerGroup = 4;  // output rows handled by one lane group
constexpr int kWaves = 4;         // waves per workgroup

template <int BITS>
__device__ __forceinline__ void load_chunk(const uint32_t* __restrict__ p, uint32_t (&w)[BITS]) {
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

// Value j (0..31) of a 32-value chunk held in BITS little-endian words.
template <int BITS>
__device__ __forceinline__ float code_at(const uint32_t (&w)[BITS], int j) {
  const int bit = j * BITS;
  const int word = bit >> 5;
  const int off = bit & 31;
  uint32_t v = w[word] >> off;
  if (off + BITS > 32) v |= w[word + 1] << (32 - off);
  return float(v & ((1u << BITS) - 1u));
}

template <int BITS, int M>
__global__ __launch_bounds__(256) void qmv_exact_kernel(
    const uint32_t* __restrict__ codes, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ y, int n, int k, int gs, int lanes_per_row) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int L = lanes_per_row;
  const int li = lane & (L - 1);
  const int lg = lane / L;
  const int groups_per_wave = 64 / L;
  const int row0 =
      ((blockIdx.x * kWaves + wave) * groups_per_wave + lg) * kRowsPerGroup;
  const int chunks = k >> 5;
  const int words_per_row = (k * BITS) >> 5;
  const int groups_per_row = k / gs;

  // Rows past the end read the last row (in bounds) and write nothing.
  int rows[kRowsPerGroup];
#pragma unroll
  for (int r = 0; r < kRowsPerGroup; ++r) rows[r] = min(row0 + r, n - 1);

  float lane_acc[M][kRowsPerGroup];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < kRowsPerGroup; ++r) lane_acc[m][r] = 0.0f;

  for (int c = li; c < chunks; c += L) {
    // Activation chunk for every row m: 32 bf16 values (64 bytes) and its sum.
    uint32_t xw[M][16];
    float sx[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* xp = reinterpret_cast<const uint4*>(x + size_t(m) * k + size_t(c) * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = xp[q];
        xw[m][4 * q + 0] = v.x; xw[m][4 * q + 1] = v.y;
        xw[m][4 * q + 2] = v.z; xw[m][4 * q + 3] = v.w;
      }
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const uint32_t d = xw[m][j >> 1];
        s = s + ((j & 1) ? u2f(d & 0xffff0000u) : u2f(d << 16));
      }
      sx[m] = s;
    }
    const int g = (c * 32) / gs;
#pragma unroll
    for (int r = 0; r < kRowsPerGroup; ++r) {
      uint32_t w[BITS];
      load_chunk<BITS>(codes + size_t(rows[r]) * words_per_row + size_t(c) * BITS, w);
      const float sc = bf16_to_f32(scales[size_t(rows[r]) * groups_per_row + g]);
      const float bi = bf16_to_f32(biases[size_t(rows[r]) * groups_per_row + g]);
      float qf[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) qf[j] = code_at<BITS>(w, j);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
          const uint32_t d = xw[m][j >> 1];
          const float xv = (j & 1) ? u2f(d & 0xffff0000u) : u2f(d << 16);
          acc = fmaf_(xv, qf[j], acc);
        }
        lane_acc[m][r] = lane_acc[m][r] + fmaf_(sc, acc, bi * sx[m]);
      }
    }
  }

  // Xor butterfly across the L lanes of the group.
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < kRowsPerGroup; ++r) {
      float v = lane_acc[m][r];
      for (int o = L >> 1; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
      lane_acc[m][r] = v;
    }
  if (li == 0) {
#pragma unroll
    for (int r = 0; r < kRowsPerGroup; ++r) {
      const int row = row0 + r;
      if (row < n) {
#pragma unroll
        for (int m = 0; m < M; ++m) y[size_t(m) * n + row] = f32_to_bf16(lane_acc[m][r]);
      }
    }
  }
}

template <int BITS, int M>
void launch_qmv(const QWeight& w, const uint16_t* x, uint16_t* y, hipStream_t s) {
  const int chunks = w.k / 32;
  int L = 1;
  while (L * 2 <= chunks && L < 64) L *= 2;
  const int rows_per_block = kWaves * (64 / L) * kRowsPerGroup;
  const int blocks = (w.n + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((qmv_exact_kernel<BITS, M>), dim3(blocks), dim3(64 * kWaves), 0, s,
                     w.codes, w.scales, w.biases, x, y, w.n, w.k, w.group_size, L);
}

template <int BITS>
void dispatch_m(const QWeight& w, const uint16_t* x, int m, uint16_t* y, hipStream_t s) {
  switch (m) {
    case 1: launch_qmv<BITS, 1>(w, x, y, s); break;
    case 2: launch_qmv<BITS, 2>(w, x, y, s); break;
    case 3: launch_qmv<BITS, 3>(w, x, y, s); break;
    case 4: launch_qmv<BITS, 4>(w, x, y, s); break;
    case 5: launch_qmv<BITS, 5>(w, x, y, s); break;
    case 6: launch_qmv<BITS, 6>(w, x, y, s); break;
    case 7: launch_qmv<BITS, 7>(w, x, y, s); break;
    default: launch_qmv<BITS, 8>(w, x, y, s); break;
  }
}

// ---- dequantisation of selected rows (embedding gather) ----
__global__ __launch_bounds__(256) void dequant_rows_kernel(
    const uint32_t* __restrict__ codes, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint32_t* __restrict__ ids,
    uint16_t* __restrict__ out, int k, int bits, int gs, int n) {
  const int i = blockIdx.y;
  const uint32_t row = min(ids[i], uint32_t(n - 1));
  const int words_per_row = (k * bits) >> 5;
  const uint32_t* rw = codes + size_t(row) * words_per_row;
  const uint32_t mask = (1u << bits) - 1u;
  for (int col = blockIdx.x * blockDim.x + threadIdx.x; col < k; col += gridDim.x * blockDim.x) {
    const int bit = col * bits;
    const int word = bit >> 5, off = bit & 31;
    uint32_t v = rw[word] >> off;
    if (off + bits > 32) v |= rw[word + 1] << (32 - off);
    const float q = float(v & mask);
    const int g = col / gs;
    const float sc = bf16_to_f32(scales[size_t(row) * (k / gs) + g]);
    const float bi = bf16_to_f32(biases[size_t(row) * (k / gs) + g]);
    // s*q is exact in fp32 (8-bit significand times an integer below 2^8),
    // so this is bf16(round_fp32(s*q + b)), matching MLX's dequantize.
    out[size_t(i) * k + col] = f32_to_bf16(sc * q + bi);
  }
}

}  // namespace

int qmv(const QWeight& w, const uint16_t* x, int m, uint16_t* y, hipStream_t s) {
  switch (w.bits) {
    case 4: dispatch_m<4>(w, x, m, y, s); break;
    case 5: dispatch_m<5>(w, x, m, y, s); break;
    case 6: dispatch_m<6>(w, x, m, y, s); break;
    case 8: dispatch_m<8>(w, x, m, y, s); break;
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int dequant_rows(const QWeight& w, const uint32_t* ids, int count, uint16_t* out, hipStream_t s) {
  if (count == 0) return MX_OK;
  const int bx = (w.k + 255) / 256;
  hipLaunchKernelGGL(dequant_rows_kernel, dim3(bx, count), dim3(256), 0, s, w.codes, w.scales,
                     w.biases, ids, out, w.k, w.bits, w.group_size, w.n);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
