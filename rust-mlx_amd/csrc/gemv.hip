// Unquantised bf16 GEMV for 1..8 activation rows (gfx950).
//
// Reference: gemv_kernel::project (src/gemv_kernel.rs:30-90) with
// kernels/shared_gemv.metal, the reference's bf16 router option: rows of one
// call share every weight load, and each row keeps the summation order of a
// single-row call, so batching does not change a row's bits.
//
// Order (restated by the CPU oracle): each output column is summed by 32 lanes;
// lane l accumulates, over k-blocks of 128 in order, values k0 + 4 l + c
// (c = 0..3) with one fma each; the 32 partial sums are combined by a
// shuffle-down tree with offsets 16, 8, 4, 2, 1; the sum is rounded to bf16.
//
// Mapping: a wave64 holds two columns, one per 32-lane half; a workgroup of
// 4 waves covers 8 columns.  Weights are read as 8-byte pieces (4 bf16 per lane
// per block, 256 contiguous bytes per half-wave); x rows are read the same way
// and stay in L1/L2 across columns.
#include "common.hpp"
#include "kernels.hpp"

namespace mx {

namespace {

template <int ROWS>
__global__ __launch_bounds__(256) void gemv_bf16_kernel(const uint16_t* __restrict__ w, int n,
                                                        int k, const uint16_t* __restrict__ x,
                                                        uint16_t* __restrict__ y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane & 31;
  const int col = blockIdx.x * 8 + wave * 2 + (lane >> 5);
  const bool live = col < n;
  const uint16_t* wr = w + size_t(live ? col : n - 1) * k + 4 * hl;
  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
  for (int k0 = 0; k0 < k; k0 += 128) {
    const uint2 wv = *reinterpret_cast<const uint2*>(wr + k0);
    const float wf[4] = {u2f(wv.x << 16), u2f(wv.x & 0xffff0000u), u2f(wv.y << 16),
                         u2f(wv.y & 0xffff0000u)};
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const uint2 xv = *reinterpret_cast<const uint2*>(x + size_t(r) * k + k0 + 4 * hl);
      const float xf[4] = {u2f(xv.x << 16), u2f(xv.x & 0xffff0000u), u2f(xv.y << 16),
                           u2f(xv.y & 0xffff0000u)};
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[r] = fmaf_(wf[c], xf[c], acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    float v = acc[r];
#pragma unroll
    for (int d = 16; d >= 1; d >>= 1) v = v + __shfl_down(v, d, 32);
    if (hl == 0 && live) y[size_t(r) * n + col] = f32_to_bf16(v);
  }
}

}  // namespace

int gemv_bf16(const uint16_t* w, int n, int k, const uint16_t* x, int rows, uint16_t* y,
              hipStream_t s) {
  if (rows < 1 || rows > 8 || n < 1 || k < 128 || k % 128 != 0) return MX_EUNSUPPORTED;
  const dim3 grid((n + 7) / 8);
  switch (rows) {
#define MX_GV(R) \
  case R: hipLaunchKernelGGL(gemv_bf16_kernel<R>, grid, dim3(256), 0, s, w, n, k, x, y); break;
    MX_GV(1) MX_GV(2) MX_GV(3) MX_GV(4) MX_GV(5) MX_GV(6) MX_GV(7) MX_GV(8)
#undef MX_GV
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
