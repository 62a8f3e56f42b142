// Affine-quantised matvec / skinny GEMM for 1..8 activation rows (gfx950),
// and row dequantisation (embedding gather).
//
// Replaces reference kernels/verify_qmv.{h,metal} (dispatched from
// src/qmv_kernel.rs:49-180) and the native quantized_matmul / gather_qmm rows
// of Linear::forward_rows (src/weights.rs:111-202).  The arithmetic order is
// the one documented in qmv_core.hpp.
#include "common.hpp"
#include "kernels.hpp"
#include "qmv_core.hpp"

namespace mx {

namespace {

constexpr int kWaves = 4;  // waves per workgroup

template <int BITS, int M>
__global__ __launch_bounds__(256) void qmv_kernel(const uint32_t* __restrict__ codes,
                                                  const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases,
                                                  const uint16_t* __restrict__ x,
                                                  uint16_t* __restrict__ y, int n, int k, int gs,
                                                  int L) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & (L - 1);
  const int lg = lane / L;
  const int row0 = ((blockIdx.x * kWaves + wave) * (64 / L) + lg) * kQRows;
  if (row0 >= n) return;  // whole lane group past the end (uniform per group)
  int rows[kQRows];
#pragma unroll
  for (int r = 0; r < kQRows; ++r) rows[r] = min(row0 + r, n - 1);
  const uint16_t* xrow[M];
#pragma unroll
  for (int m = 0; m < M; ++m) xrow[m] = x + size_t(m) * k;
  float out[M][kQRows];
  qmv_core<BITS, M>(codes, scales, biases, k, gs, xrow, rows, li, L, out);
  if (li == 0) {
#pragma unroll
    for (int r = 0; r < kQRows; ++r)
      if (row0 + r < n)
#pragma unroll
        for (int m = 0; m < M; ++m) y[size_t(m) * n + row0 + r] = f32_to_bf16(out[m][r]);
  }
}

template <int BITS, int M>
void launch_qmv(const QWeight& w, const uint16_t* x, uint16_t* y, hipStream_t s) {
  const int L = qmv_lanes_per_row(w.k);
  const int rows_per_block = kWaves * (64 / L) * kQRows;
  const int blocks = (w.n + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((qmv_kernel<BITS, M>), dim3(blocks), dim3(64 * kWaves), 0, s, w.codes,
                     w.scales, w.biases, x, y, w.n, w.k, w.group_size, L);
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
  // Out-of-range ids are clamped to the last row; hosts validate token ids.
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
