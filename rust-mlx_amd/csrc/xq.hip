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

#define MX_TRY_RC(x)              \
  do {                            \
    const int rc_ = (x);          \
    if (rc_ != MX_OK) return rc_; \
  } while (0)

namespace mx {

namespace {

constexpr int kXqStageGroups = 64;  // groups staged in LDS (K <= 4096)

struct XRows {
  const uint16_t* x;
  int64_t stride;
  __device__ __forceinline__ const uint16_t* operator()(int m) const { return x + m * stride; }
};

template <class F>
int raise_lds(F fn, int lb) {
  // stagings above the default 64 KiB of dynamic LDS need the attribute
  if (lb > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, lb) != hipSuccess)
    return MX_EHIP;
  return MX_OK;
}

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

// The projection values of one workgroup: wave (t, ks) streams the weight
// row of its lane (crow / srow / brow: tile t's row l % 16) over slice ks's
// groups against activation rows xr(0..M-1) (staged in LDS, or built in
// registers when XREG), and yt[m][t * 16 + j] receives the fp32 result of
// activation row m and tile row j.  `pre` runs once the slice's weight loads
// are issued (the caller's own prefetches).  Ends with a barrier.
template <int BITS, int T, int KS, bool XREG, class Rows, class Pre>
__device__ __forceinline__ void xq_tiles(const uint32_t* __restrict__ crow,
                                         const uint16_t* __restrict__ srow,
                                         const uint16_t* __restrict__ brow, int K, int M,
                                         const Rows& xr, char* lds, double* red, float* yt,
                                         Pre&& pre) {
  constexpr int NC = 16 * T, NT = 64 * T * KS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, kb = lane >> 4;
  const int t = wave / KS, ks = wave - t * KS;
  const int G = K / xq::kGroup, gps = G / KS, g0 = ks * gps;
  // the slice's code words, scales and biases, all issued up front
  xq::Codes<BITS> c[xq::kGroupsPerSlice];
  uint16_t sv[xq::kGroupsPerSlice], bv[xq::kGroupsPerSlice];
#pragma unroll
  for (int i = 0; i < xq::kGroupsPerSlice; ++i) {
    const int g = g0 + min(i, gps - 1);
    xq::load_codes<BITS>(crow, g, kb, c[i]);
    sv[i] = srow[g];
    bv[i] = brow[g];
  }
  pre();
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
}

// Dense projections (modes of ProjEpilogue).  Workgroup tg covers rows
// tg*16T .. tg*16T + 16T - 1 (tile t: rows tg*16T + 16t + j); for kHcUpMix
// (T = 4) it covers columns tg*16 .. tg*16 + 15 of the four streams (tile t:
// rows t*H + tg*16 + j).
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
  const int j = threadIdx.x & 15, t = (threadIdx.x >> 6) / KS;
  const int n = w.n, G = w.k / xq::kGroup;
  int row;
  if constexpr (MODE == kHcUpMix)
    row = t * e.hidden + min(tg * 16 + j, e.hidden - 1);
  else
    row = min(tg * NC + t * 16 + j, n - 1);
  ProjFinish<MODE, NC, NT> fin;
  fin.begin(e, tg, M, n);
  xq_tiles<BITS, T, KS, XREG>(w.codes + size_t(row) * (size_t(w.k) * BITS / 32),
                              w.scales + size_t(row) * G, w.biases + size_t(row) * G, w.k, M,
                              XRows{x, x_stride}, lds, red, yt, [&] { fin.prefetch(e); });
  fin.finish(yt, e, tg, M, n);
}

// Activation rows of an expert plan entry: member m is route (row, slot) at
// base + row * row_stride + slot * slot_stride.
struct MemberRows {
  const uint16_t* base;
  int64_t row_stride, slot_stride;
  const int* ro;
  const int* so;
  __device__ __forceinline__ const uint16_t* operator()(int m) const {
    return base + ro[m] * row_stride + so[m] * slot_stride;
  }
};

// Bank matrix of one expert (expert < 0: the shared expert's matrix).
__device__ __forceinline__ QWeight bank_matrix(const QBank& b, int expert, const QWeight& shared) {
  if (expert < 0) return shared;
  const size_t cs = size_t(b.n) * b.k * b.bits / 32;
  const size_t ss = size_t(b.n) * (b.k / b.group_size);
  return QWeight{b.codes + cs * expert, b.scales + ss * expert, b.biases + ss * expert, b.n, b.k,
                 b.bits, b.group_size};
}

// Expert gate/up + SwiGLU for one plan entry (blockIdx.y) and 32
// intermediate rows (blockIdx.x): tiles 0-1 are gate rows, tiles 2-3 the same
// up rows; h[row][slot][i] = bf16(bf16(silu(bf16(g))) * bf16(u)) for the
// entry's member routes (the exact kernels' SwiGLU, moe.hip gate_up_body).
template <int BITS, int KS>
__global__ __launch_bounds__(64 * 4 * KS) void xq_gate_up_kernel(
    const uint16_t* __restrict__ x, const MoePlan* __restrict__ plan, int top_k, QBank gate,
    QBank up, QWeight sgate, QWeight sup, uint16_t* __restrict__ h, int hs) {
  extern __shared__ __align__(16) char lds[];
  __shared__ double red[KS * 4 * 8 * 16];
  __shared__ float yt[8 * 64];
  __shared__ int ro[8], so[8];
  const int entry = blockIdx.y;
  if (entry >= plan->count) return;
  const int expert = plan->expert[entry];
  const QWeight gw = bank_matrix(gate, expert, sgate);
  const QWeight uw = bank_matrix(up, expert, sup);
  const int inter = gw.n, hidden = gw.k;
  const int i0 = blockIdx.x * 32;
  if (i0 >= inter) return;
  const int M = plan->m[entry];
  if (threadIdx.x < 8) {
    ro[threadIdx.x] = plan->row[entry][threadIdx.x];
    so[threadIdx.x] = plan->slot[entry][threadIdx.x];
  }
  __syncthreads();
  const int j = threadIdx.x & 15, t = (threadIdx.x >> 6) / KS;
  const QWeight& mw = t < 2 ? gw : uw;
  const int row = min(i0 + 16 * (t & 1) + j, inter - 1);
  const int G = hidden / xq::kGroup;
  xq_tiles<BITS, 4, KS, false>(mw.codes + size_t(row) * (size_t(hidden) * BITS / 32),
                               mw.scales + size_t(row) * G, mw.biases + size_t(row) * G, hidden,
                               M, MemberRows{x, hidden, 0, ro, so}, lds, red, yt, [] {});
  for (int i = threadIdx.x; i < 8 * 32; i += 64 * 4 * KS) {
    const int m = i >> 5, c = i & 31;
    if (m >= M || i0 + c >= inter) continue;
    const float gv = round_bf16(yt[m * 64 + c]);
    const float uv = round_bf16(yt[m * 64 + 32 + c]);
    const float silu = round_bf16(gv * sigmoid_bf16(gv));
    h[(size_t(ro[m]) * (top_k + 1) + so[m]) * hs + i0 + c] = f32_to_bf16(silu * uv);
  }
}

// Expert down + route score for one plan entry (blockIdx.y) and 64 output
// columns (blockIdx.x): p[row][slot][c] = bf16(bf16(down h) * score) for
// routed slots, bf16(down h) for the shared slot (moe.hip down_body).
template <int BITS, int KS>
__global__ __launch_bounds__(64 * 4 * KS) void xq_down_kernel(
    const uint16_t* __restrict__ h, const MoePlan* __restrict__ plan,
    const uint16_t* __restrict__ scores, int top_k, QBank down, QWeight sdown,
    uint16_t* __restrict__ p, int hs) {
  extern __shared__ __align__(16) char lds[];
  __shared__ double red[KS * 4 * 8 * 16];
  __shared__ float yt[8 * 64];
  __shared__ int ro[8], so[8];
  const int entry = blockIdx.y;
  if (entry >= plan->count) return;
  const int expert = plan->expert[entry];
  const QWeight dw = bank_matrix(down, expert, sdown);
  const int hidden = dw.n, inter = dw.k;
  const int c0 = blockIdx.x * 64;
  if (c0 >= hidden) return;
  const int M = plan->m[entry];
  if (threadIdx.x < 8) {
    ro[threadIdx.x] = plan->row[entry][threadIdx.x];
    so[threadIdx.x] = plan->slot[entry][threadIdx.x];
  }
  __syncthreads();
  const int j = threadIdx.x & 15, t = (threadIdx.x >> 6) / KS;
  const int row = min(c0 + 16 * t + j, hidden - 1);
  const int G = inter / xq::kGroup;
  xq_tiles<BITS, 4, KS, false>(dw.codes + size_t(row) * (size_t(inter) * BITS / 32),
                               dw.scales + size_t(row) * G, dw.biases + size_t(row) * G, inter,
                               M, MemberRows{h, int64_t(top_k + 1) * hs, hs, ro, so}, lds, red, yt,
                               [] {});
  for (int i = threadIdx.x; i < 8 * 64; i += 64 * 4 * KS) {
    const int m = i >> 6, c = i & 63;
    if (m >= M || c0 + c >= hidden) continue;
    const bool routed = so[m] < top_k;
    const float dv = round_bf16(yt[i]);
    const float sc = routed ? bf16_to_f32(scores[size_t(ro[m]) * top_k + so[m]]) : 1.0f;
    p[(size_t(ro[m]) * (top_k + 1) + so[m]) * hidden + c0 + c] = f32_to_bf16(routed ? dv * sc : dv);
  }
}

__device__ __forceinline__ void better_of(float v, uint32_t id, float& best, uint32_t& best_id) {
  if (v > best || (v == best && id < best_id)) {
    best = v;
    best_id = id;
  }
}

// Greedy head: per activation row, the best (bf16 logit, lowest id) of the
// workgroup's 64 vocabulary rows (NaN never wins; nothing above -inf keeps id
// 0xffffffff), and, when asked, the bf16 logits themselves.
template <int BITS, int KS>
__global__ __launch_bounds__(64 * 4 * KS) void xq_head_kernel(QWeight w,
                                                              const uint16_t* __restrict__ x,
                                                              int M, float* __restrict__ maxima,
                                                              uint32_t* __restrict__ indices,
                                                              uint16_t* __restrict__ logits) {
  extern __shared__ __align__(16) char lds[];
  __shared__ double red[KS * 4 * 8 * 16];
  __shared__ float yt[8 * 64];
  const int tg = blockIdx.x, parts = gridDim.x;
  const int j = threadIdx.x & 15, t = (threadIdx.x >> 6) / KS;
  const int n = w.n, G = w.k / xq::kGroup;
  const int row = min(tg * 64 + 16 * t + j, n - 1);
  xq_tiles<BITS, 4, KS, false>(w.codes + size_t(row) * (size_t(w.k) * BITS / 32),
                               w.scales + size_t(row) * G, w.biases + size_t(row) * G, w.k, M,
                               XRows{x, w.k}, lds, red, yt, [] {});
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int m = wave; m < M; m += 4 * KS) {
    const int r = tg * 64 + lane;
    float best = u2f(0xff800000u);
    uint32_t best_id = 0xffffffffu;
    if (r < n) {
      better_of(round_bf16(yt[m * 64 + lane]), uint32_t(r), best, best_id);
      if (logits) logits[size_t(m) * n + r] = f32_to_bf16(yt[m * 64 + lane]);
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float v = __shfl_xor(best, o, 64);
      const uint32_t id = uint32_t(__shfl_xor(int(best_id), o, 64));
      better_of(v, id, best, best_id);
    }
    if (lane == 0) {
      maxima[size_t(m) * parts + tg] = best;
      indices[size_t(m) * parts + tg] = best_id;
    }
  }
}

template <int BITS, int MODE, int T, int KS, bool XREG>
int launch_xq(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
              hipStream_t s) {
  const int groups = MODE == kHcUpMix ? (e.hidden + 15) / 16 : (w.n + 16 * T - 1) / (16 * T);
  const int lb = XREG ? 0 : xq::stage_bytes(w.k / xq::kGroup);
  const auto fn = xq_dense_kernel<BITS, MODE, T, KS, XREG>;
  MX_TRY_RC(raise_lds(fn, lb));
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

template <int BITS, int KS>
int launch_gate_up(const uint16_t* x, const MoePlan* plan, int routes, int top_k,
                   const QBank& gate, const QBank& up, const QWeight& sgate, const QWeight& sup,
                   uint16_t* h, int hs, hipStream_t s) {
  const auto fn = xq_gate_up_kernel<BITS, KS>;
  const int lb = xq::stage_bytes(gate.k / xq::kGroup);
  MX_TRY_RC(raise_lds(fn, lb));
  hipLaunchKernelGGL(fn, dim3((hs + 31) / 32, routes), dim3(64 * 4 * KS), lb, s, x, plan, top_k,
                     gate, up, sgate, sup, h, hs);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

template <int BITS, int KS>
int launch_down(const uint16_t* h, const MoePlan* plan, int routes, const uint16_t* scores,
                int top_k, const QBank& down, const QWeight& sdown, uint16_t* p, int hs,
                hipStream_t s) {
  const auto fn = xq_down_kernel<BITS, KS>;
  const int kmax = down.k > sdown.k ? down.k : sdown.k;
  const int lb = xq::stage_bytes(kmax / xq::kGroup);
  MX_TRY_RC(raise_lds(fn, lb));
  hipLaunchKernelGGL(fn, dim3((down.n + 63) / 64, routes), dim3(64 * 4 * KS), lb, s, h, plan,
                     scores, top_k, down, sdown, p, hs);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

template <int BITS, int KS>
int launch_head(const QWeight& w, const uint16_t* x, int m, float* maxima, uint32_t* indices,
                uint16_t* logits, int parts, hipStream_t s) {
  const auto fn = xq_head_kernel<BITS, KS>;
  const int lb = xq::stage_bytes(w.k / xq::kGroup);
  MX_TRY_RC(raise_lds(fn, lb));
  hipLaunchKernelGGL(fn, dim3(parts), dim3(64 * 4 * KS), lb, s, w, x, m, maxima, indices, logits);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

// Expert matrices take K in {64 .. 512} (one slice), 1024 or 2048.
bool xq_bank_ok(int k) { return (k % 64 == 0 && k <= 512) || k == 1024 || k == 2048; }

}  // namespace

int xq_gate_up(const uint16_t* x, const MoePlan* plan, int rows, int top_k, const QBank& gate,
               const QBank& up, const QWeight& sgate, const QWeight& sup, uint16_t* h,
               hipStream_t s) {
  if (gate.group_size != 64 || up.group_size != 64 || sgate.group_size != 64 ||
      sup.group_size != 64 || !xq_bank_ok(gate.k) || sgate.k != gate.k || up.k != gate.k ||
      gate.bits != up.bits || sgate.bits != gate.bits || sup.bits != gate.bits)
    return MX_EUNSUPPORTED;
  const int routes = rows * top_k + 1;
  const int hs = gate.n > sgate.n ? gate.n : sgate.n;
  const int ks = xq::slices(gate.k);
#define MX_GU(B, K_) \
  if (gate.bits == B && ks == K_) return launch_gate_up<B, K_>(x, plan, routes, top_k, gate, up, sgate, sup, h, hs, s);
  MX_GU(4, 1) MX_GU(4, 2) MX_GU(4, 4) MX_GU(5, 1) MX_GU(5, 2) MX_GU(5, 4)
  MX_GU(6, 1) MX_GU(6, 2) MX_GU(6, 4) MX_GU(8, 1) MX_GU(8, 2) MX_GU(8, 4)
#undef MX_GU
  return MX_EUNSUPPORTED;
}

int xq_down(const uint16_t* h, const MoePlan* plan, const uint16_t* scores, int rows, int top_k,
            int inter, int shared_inter, const QBank& down, const QWeight& sdown, uint16_t* p,
            hipStream_t s) {
  if (down.group_size != 64 || sdown.group_size != 64 || !xq_bank_ok(down.k) ||
      !xq_bank_ok(sdown.k) || xq::slices(down.k) != xq::slices(sdown.k) ||
      sdown.bits != down.bits || sdown.n != down.n)
    return MX_EUNSUPPORTED;
  const int routes = rows * top_k + 1;
  const int hs = inter > shared_inter ? inter : shared_inter;
  const int ks = xq::slices(down.k);
#define MX_DN(B, K_) \
  if (down.bits == B && ks == K_) return launch_down<B, K_>(h, plan, routes, scores, top_k, down, sdown, p, hs, s);
  MX_DN(4, 1) MX_DN(4, 2) MX_DN(4, 4) MX_DN(5, 1) MX_DN(5, 2) MX_DN(5, 4)
  MX_DN(6, 1) MX_DN(6, 2) MX_DN(6, 4) MX_DN(8, 1) MX_DN(8, 2) MX_DN(8, 4)
#undef MX_DN
  return MX_EUNSUPPORTED;
}

int xq_head_parts(int n) { return (n + 63) / 64; }

int xq_head(const QWeight& w, const uint16_t* x, int m, float* maxima, uint32_t* indices,
            uint16_t* logits, int* parts_out, hipStream_t s) {
  if (w.group_size != 64 || !xq_bank_ok(w.k) || m < 1 || m > 8) return MX_EUNSUPPORTED;
  const int parts = xq_head_parts(w.n);
  *parts_out = parts;
  const int ks = xq::slices(w.k);
#define MX_HD(B, K_) \
  if (w.bits == B && ks == K_) return launch_head<B, K_>(w, x, m, maxima, indices, logits, parts, s);
  MX_HD(4, 1) MX_HD(4, 2) MX_HD(4, 4) MX_HD(5, 1) MX_HD(5, 2) MX_HD(5, 4)
  MX_HD(6, 1) MX_HD(6, 2) MX_HD(6, 4) MX_HD(8, 1) MX_HD(8, 2) MX_HD(8, 4)
#undef MX_HD
  return MX_EUNSUPPORTED;
}

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
