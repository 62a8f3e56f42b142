// Exact-integer projections for 1..8 activation rows (the arithmetic of
// xq_core.hpp): dense projections with the engine's fused epilogues.
//
// Replaces the same reference interfaces as the other projection kernels:
// the QMV / gather_qmm rows of Linear::forward_rows (src/weights.rs:111-202,
// src/qmv_kernel.rs:49-180).  Results equal the CPU oracle's mxo_xq bit for
// bit: every integer sum is exact and the fp64 group combination follows the
// oracle's slice order, so neither the tile shape nor the number of rows
// changes a bit.
//
// A workgroup holds T tiles of 16 weight rows; wave (t, ks) of a tile runs
// slice ks of the row's groups (the slices of the arithmetic, so KS is fixed
// by K).  For K <= 4096 the activation rows are staged once per workgroup in
// LDS as int8 digit operands (the slice's weight loads are issued first, so
// both latencies overlap); deeper rows build each wave's operands in
// registers.  The KS slice sums of a tile are added in slice order in LDS.
#include "common.hpp"
#include "kernels.hpp"
#include "proj_epilogue.hpp"
#include "xq_core.hpp"

namespace mx {

namespace {

constexpr int kXqStageGroups = 64;  // groups staged in LDS (K <= 4096)

struct XRows {
  const uint16_t* x;
  int64_t stride;
  __device__ __forceinline__ const uint16_t* operator()(int m) const { return x + m * stride; }
};

// Register-built A operand of one group for this lane (XREG): block bk's row
// r = 4 bk + (l % 16) / 4, digit l % 4, values 16 (l / 16) .. +15 in
// perm<BITS>() order; q and eb of the row this lane supplies.
template <int BITS>
__device__ __forceinline__ xq::v4i reg_operand(const XRows& xr, int M, int bk, int g, double& q,
                                               int& eb) {
  const int lane = threadIdx.x & 63, kb = lane >> 4, d = lane & 3;
  const int r = 4 * bk + ((lane & 15) >> 2);
  float f[16];
  if (r < M) {
    const uint4* src = reinterpret_cast<const uint4*>(xr(r) + size_t(g) * xq::kGroup + 16 * kb);
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
  eb = max(int((f2u(amax) >> 23) & 0xffu), 1);
  eb = max(eb, __shfl_xor(eb, 16, 64));
  eb = max(eb, __shfl_xor(eb, 32, 64));
  int X[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) X[i] = xq::grid_int(f[i], eb);
  q = 0.0;
#pragma unroll
  for (int i = 0; i < 8; ++i) q += double(X[2 * i] + X[2 * i + 1]);
  q += __shfl_xor(q, 16, 64);
  q += __shfl_xor(q, 32, 64);
  const uint32_t sh = 8u * uint32_t(d);
  uint32_t o[4];
#pragma unroll
  for (int pw = 0; pw < 4; ++pw) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v |= ((xq::digits(X[xq::perm<BITS>(4 * pw + i)]) >> sh) & 0xffu) << (8 * i);
    o[pw] = v;
  }
  xq::v4i op;
  op.x = int(o[0]); op.y = int(o[1]); op.z = int(o[2]); op.w = int(o[3]);
  return op;
}

template <int BITS, int MODE, int T, int KS, bool XREG>
__global__ __launch_bounds__(64 * T * KS) void xq_dense_kernel(QWeight w,
                                                               const uint16_t* __restrict__ x,
                                                               int64_t x_stride, int M,
                                                               ProjEpilogue e) {
  extern __shared__ __align__(16) char lds[];
  __shared__ double red[KS * T * 8 * 16];
  __shared__ float yt[8 * 16 * T];
  constexpr int NC = 16 * T, NT = 64 * T * KS;
  const int tg = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, kb = lane >> 4;
  const int t = wave / KS, ks = wave - t * KS;
  const int n = w.n, G = w.k / xq::kGroup, gps = G / KS, g0 = ks * gps;
  int row;
  if constexpr (MODE == kHcUpMix)
    row = t * e.hidden + min(tg * 16 + j, e.hidden - 1);
  else
    row = min(tg * NC + t * 16 + j, n - 1);
  ProjFinish<MODE, NC, NT> fin;
  fin.begin(e, tg, M, n);
  // the slice's code words, scales and biases, all issued up front
  const uint32_t* crow = w.codes + size_t(row) * (size_t(w.k) * BITS / 32);
  xq::Codes<BITS> c[xq::kGroupsPerSlice];
  uint16_t sv[xq::kGroupsPerSlice], bv[xq::kGroupsPerSlice];
#pragma unroll
  for (int i = 0; i < xq::kGroupsPerSlice; ++i) {
    const int g = g0 + min(i, gps - 1);
    xq::load_codes<BITS>(crow, g, kb, c[i]);
    sv[i] = w.scales[size_t(row) * G + g];
    bv[i] = w.biases[size_t(row) * G + g];
  }
  fin.prefetch(e);
  const XRows xr{x, x_stride};
  const bool two = M > 4;
  double acc[2] = {0.0, 0.0};
  if constexpr (!XREG) {
    xq::stage<BITS, NT>(lds, xr, M, 0, G);
    const double* qs = reinterpret_cast<const double*>(lds + G * xq::kGroupBytes);
    const int* es = reinterpret_cast<const int*>(lds + G * (xq::kGroupBytes + 64));
#pragma unroll
    for (int i = 0; i < xq::kGroupsPerSlice; ++i) {
      if (i < gps) {
        const int g = g0 + i;
        const char* ab = lds + g * xq::kGroupBytes + lane * 16;
        const xq::v4i a0 = *reinterpret_cast<const xq::v4i*>(ab);
        const xq::v4i a1 = *reinterpret_cast<const xq::v4i*>(ab + xq::kBlockBytes);
        xq::group_step<BITS>(a0, a1, two, xq::b_operand<BITS>(c[i]), qs[g * 8 + kb],
                             qs[g * 8 + 4 + kb], es[g * 8 + kb], es[g * 8 + 4 + kb],
                             double(bf16_to_f32(sv[i])), double(bf16_to_f32(bv[i])), acc);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < xq::kGroupsPerSlice; ++i) {
      if (i < gps) {
        const int g = g0 + i;
        double q0, q1 = 0.0;
        int e0, e1 = 1;
        const xq::v4i a0 = reg_operand<BITS>(xr, M, 0, g, q0, e0);
        xq::v4i a1 = {0, 0, 0, 0};
        if (two) a1 = reg_operand<BITS>(xr, M, 1, g, q1, e1);
        // this lane receives activation row kb of each block: the Q and Eb
        // of that row sit in the lanes that supplied it (l % 16 = 4 kb)
        const int src = 4 * kb;
        const double rq0 = __shfl(q0, src, 64), rq1 = __shfl(q1, src, 64);
        const int re0 = __shfl(e0, src, 64), re1 = __shfl(e1, src, 64);
        xq::group_step<BITS>(a0, a1, two, xq::b_operand<BITS>(c[i]), rq0, rq1, re0, re1,
                             double(bf16_to_f32(sv[i])), double(bf16_to_f32(bv[i])), acc);
      }
    }
  }
  // slice sums in slice order, from +0, then one rounding to fp32
  red[((ks * T + t) * 8 + kb) * 16 + j] = acc[0];
  red[((ks * T + t) * 8 + 4 + kb) * 16 + j] = acc[1];
  __syncthreads();
  for (int i = threadIdx.x; i < 8 * NC; i += NT) {
    const int m = i / NC, cc = i - m * NC;
    const int tt = cc >> 4, jj = cc & 15;
    double total = 0.0;
#pragma unroll
    for (int k = 0; k < KS; ++k) total = total + red[((k * T + tt) * 8 + m) * 16 + jj];
    yt[i] = float(total);
  }
  __syncthreads();
  fin.finish(yt, e, tg, M, n);
}

template <int BITS, int MODE, int T, int KS, bool XREG>
int launch_xq(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
              hipStream_t s) {
  const int groups = MODE == kHcUpMix ? (e.hidden + 15) / 16 : (w.n + 16 * T - 1) / (16 * T);
  const int lb = XREG ? 0 : xq::stage_bytes(w.k / xq::kGroup);
  const auto fn = xq_dense_kernel<BITS, MODE, T, KS, XREG>;
  if (lb > 65536) {
    // stagings of K > 2048 use more than the default 64 KiB of dynamic LDS
    static bool raised = false;
    if (!raised) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lb) != hipSuccess)
        return MX_EHIP;
      raised = true;
    }
  }
  hipLaunchKernelGGL(fn, dim3(groups), dim3(64 * T * KS), lb, s, w, x, xs, m, e);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

// Slices are fixed by K; tiles per workgroup fill up to 16 waves (kHcUpMix
// always takes the four streams as four tiles).
template <int BITS, int MODE>
int xq_shape(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
             hipStream_t s) {
  const int KS = xq::slices(w.k);
  const bool xreg = w.k / xq::kGroup > kXqStageGroups;
#define MX_XQ(T_, KS_, X_)                                                   \
  if (KS == KS_ && xreg == X_) return launch_xq<BITS, MODE, T_, KS_, X_>(w, x, xs, m, e, s);
  if constexpr (MODE == kHcUpMix) {
    MX_XQ(4, 1, false) MX_XQ(4, 2, false) MX_XQ(4, 4, false)
  } else {
    MX_XQ(4, 1, false) MX_XQ(4, 2, false) MX_XQ(4, 3, false) MX_XQ(4, 4, false)
    MX_XQ(2, 5, false) MX_XQ(2, 6, false) MX_XQ(2, 7, false) MX_XQ(2, 8, false)
    MX_XQ(1, 16, true) MX_XQ(1, 12, true) MX_XQ(1, 10, true) MX_XQ(1, 9, true)
  }
#undef MX_XQ
  return MX_EUNSUPPORTED;
}

template <int BITS>
int xq_mode(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
            hipStream_t s) {
  switch (e.mode) {
    case kPlain: return xq_shape<BITS, kPlain>(w, x, xs, m, e, s);
    case kHcDown: return xq_shape<BITS, kHcDown>(w, x, xs, m, e, s);
    case kHcUpMix: return xq_shape<BITS, kHcUpMix>(w, x, xs, m, e, s);
    case kConv: return xq_shape<BITS, kConv>(w, x, xs, m, e, s);
    default: return xq_shape<BITS, kHcWrite>(w, x, xs, m, e, s);
  }
}

}  // namespace

// Group size 64; K a multiple of 64 up to 512, or a multiple of 512 up to
// 8192 (slices of eight groups); 16-byte aligned activation rows.
bool xq_supported(const QWeight& w) {
  const int ks = xq::slices(w.k);
  const bool shape = (w.k % 64 == 0 && w.k <= 512) ||
                     (w.k % 512 == 0 && (ks <= 10 || ks == 12 || ks == 16));
  return w.group_size == 64 && shape && (w.bits == 4 || w.bits == 5 || w.bits == 6 || w.bits == 8);
}

int xq_dense(const QWeight& w, const uint16_t* x, int64_t x_stride, int m, const ProjEpilogue& e,
             hipStream_t s) {
  if (!xq_supported(w) || m < 1 || m > 8) return MX_EUNSUPPORTED;
  if (e.mode == kHcUpMix && e.hidden * 4 != w.n) return MX_EUNSUPPORTED;
  if (e.mode == kConv && (e.taps < 2 || e.taps > kConvMaxTaps)) return MX_EUNSUPPORTED;
  switch (w.bits) {
    case 4: return xq_mode<4>(w, x, x_stride, m, e, s);
    case 5: return xq_mode<5>(w, x, x_stride, m, e, s);
    case 6: return xq_mode<6>(w, x, x_stride, m, e, s);
    default: return xq_mode<8>(w, x, x_stride, m, e, s);
  }
}

}  // namespace mx
