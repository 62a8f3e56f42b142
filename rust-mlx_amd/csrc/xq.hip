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

// Register-built A operand of one group for this lane (operands from
// registers): block bk's row r = 4 bk + (l % 16) / 4, digit l % 4, values
// 16 (l / 16) .. +15 in perm() order; q and eb of the row this lane supplies.
template <class Rows>
__device__ __forceinline__ xq::v4i reg_operand(const Rows& xr, int M, int bk, int g, double& q,
                                               int& eb) {
  const int lane = threadIdx.x & 63, kb = lane >> 4, d = lane & 3;
  const int r = 4 * bk + ((lane & 15) >> 2);
  float f[16];
  if (r < M) {
    xq::load16(xr(r) + size_t(g) * xq::kGroup + 16 * kb, f);
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
    for (int i = 0; i < 4; ++i) v |= ((xq::digits(X[xq::perm(4 * pw + i)]) >> sh) & 0xffu) << (8 * i);
    o[pw] = v;
  }
  xq::v4i op;
  op.x = int(o[0]); op.y = int(o[1]); op.z = int(o[2]); op.w = int(o[3]);
  return op;
}

// Where a kernel's activation operands come from.
enum : int {
  kSrcStage = 0,     // staged by the workgroup into LDS from the bf16 rows
  kSrcReg = 1,       // built by each wave in registers (deep rows, no plane)
  kSrcPlane = 2,     // read by each wave from the producer's plane in global memory
  kSrcPlaneLds = 3,  // the producer's plane copied once per workgroup into LDS
  kSrcBlockLds = 4,  // one four-row block of the plane copied into LDS (blockIdx.y)
  kSrcBlockPlane = 5,  // one four-row block of the plane read in place by each wave
};

template <int BITS>
constexpr int batch_groups() {
  return BITS == 8 ? 4 : 8;  // groups per load batch (8-bit codes are twice as wide)
}

// Groups per load batch of a wave covering 2 SPW groups.
template <int BITS, int SPW>
constexpr int tile_batch() {
  return 2 * SPW < batch_groups<BITS>() ? 2 * SPW : batch_groups<BITS>();
}

// sb_vector_ok for the batches of xq_tiles over matrix w.
template <int BITS, int SPW>
__device__ __forceinline__ bool tiles_sbv(const QWeight& w) {
  return xq::sb_vector_ok<tile_batch<BITS, SPW>()>(w.scales, w.biases, w.k / xq::kGroup);
}

// LDS bytes of xq_tiles: the staged or copied operands of G groups, and the
// slice sums of T tiles when KS > 1 (they reuse the operand area).
__host__ __device__ constexpr int tiles_lds(int G, int T, int KS, int SRC) {
  const int ops = (SRC == kSrcStage || SRC == kSrcPlaneLds) ? xq::stage_bytes(G)
                  : SRC == kSrcBlockLds                       ? xq::block_bytes(G)
                                                              : 0;
  const int sums = KS > 1 ? ((G + 1) / 2) * T * 8 * 16 * 8 : 0;
  const int b = ops > sums ? ops : sums;
  return b > 16 ? b : 16;
}

// The weight row read by a lane in row-major order (lane 4 r + q: row r of
// its tile), for the RM form of xq_tiles.
struct RmRows {
  const uint32_t* codes = nullptr;
  const uint16_t* scales = nullptr;
  const uint16_t* biases = nullptr;
};

// The projection values of one workgroup.  Wave (t, ks) streams the weight
// row of its lane (crow / srow / brow: tile t's row l % 16) over slices
// [ks SPW, ks SPW + SPW) (two groups each) against activation rows
// xr(0..M-1), in load batches kept two deep; `blocks` says which four-row
// blocks of activation rows to compute (bit 0: rows 0-3, bit 1: rows 4-7).
// With KS == 1 the wave adds its slice sums in order itself; otherwise the
// slice sums meet in LDS and are added in slice order.  yt[m][t * 16 + j]
// receives the fp32 result of activation row m and tile row j.  `pre` runs
// once the first weight loads are issued.  Ends with a barrier.
// RM (4-bit codes, batches of an even number of groups; the launcher checks
// that every wave's groups are whole batches and the scale/bias rows
// aligned): the weight stream is read in row-major lane order through `rm`
// (lane 4 r + q: 16 bytes of row r, piece q of a pair of groups, and the
// scale and bias words of groups 2q, 2q + 1 of the batch), so each four
// adjacent lanes read
// contiguous bytes, and ds_bpermute hands lane 16 kb + j the words that
// load_codes / load_scale_bias would have read for row j: the products are
// unchanged.
template <int BITS, int T, int KS, int SPW, int SRC, bool RM = false, class Rows, class Pre>
__device__ __forceinline__ void xq_tiles(const uint32_t* __restrict__ crow,
                                         const uint16_t* __restrict__ srow,
                                         const uint16_t* __restrict__ brow, bool sbv, int K,
                                         int M, int blocks, const Rows& xr, const char* plane,
                                         char* lds, float* yt, Pre&& pre,
                                         const RmRows& rm = RmRows{}) {
  constexpr int NC = 16 * T, NT = 64 * T * KS;
  constexpr int NG = 2 * SPW;
  constexpr int B = tile_batch<BITS, SPW>();
  constexpr int NB = NG / B;
  // 4-bit: pairs of groups per 16-byte piece; 8-bit: one group's 16 bytes
  // per lane, so the move is a pure lane permutation
  // 5 / 6-bit (RG): lane 4 r + q reads the code window load_codes gives
  // row r and k-block q (adjacent lanes: contiguous bytes of one row), then
  // the window's words move to lane 16 q + r
  constexpr bool RG = RM && (BITS == 5 || BITS == 6) && B % 2 == 0;
  constexpr bool R = RM && ((BITS == 4 && B % 2 == 0) || BITS == 8 || RG);
  const int lane = threadIdx.x & 63, j = lane & 15, kb = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = wave / KS, ks = wave - t * KS;
  const int G = K / xq::kGroup, S = (G + 1) / 2;
  const int gbeg = 2 * ks * SPW, gend = min(gbeg + NG, G);
  const int q4 = lane & 3;
  xq::Codes<BITS> c[R ? 1 : 2][B];
  xq::ScaleBias<B> sb[R ? 1 : 2];
  constexpr int NP = BITS == 8 ? B : (B / 2 > 0 ? B / 2 : 1);  // 16-byte pieces per batch
  uint4 rc[R && !RG ? 2 : 1][NP];
  xq::Codes<BITS> rw[RG ? 2 : 1][RG ? B : 1];
  uint32_t rs[R ? 2 : 1], rb[R ? 2 : 1];
  auto load_batch = [&](int buf, int bi) {
    if constexpr (R) {
      const int g0 = gbeg + bi * B;
#pragma unroll
      for (int pp = 0; pp < (RG ? 0 : NP); ++pp) {
        if constexpr (BITS == 8)  // piece q of group g0 + pp
          rc[buf][pp] = *reinterpret_cast<const uint4*>(rm.codes + 16 * (g0 + pp) + 4 * q4);
        else  // piece q of groups g0 + 2 pp, + 1
          rc[buf][pp] = *reinterpret_cast<const uint4*>(rm.codes + 8 * (g0 + 2 * pp) + 4 * q4);
      }
      if constexpr (RG) {
#pragma unroll
        for (int i = 0; i < B; ++i) xq::load_codes<BITS>(rm.codes, g0 + i, q4, rw[buf][i]);
      }
      // B / 2 scale (bias) words per row; lanes past them repeat the last
      const int qw = q4 & (B / 2 > 0 ? B / 2 - 1 : 0);
      rs[buf] = *reinterpret_cast<const uint32_t*>(rm.scales + g0 + 2 * qw);
      rb[buf] = *reinterpret_cast<const uint32_t*>(rm.biases + g0 + 2 * qw);
    } else {
#pragma unroll
      for (int i = 0; i < B; ++i)
        xq::load_codes<BITS>(crow, min(gbeg + bi * B + i, gend - 1), kb, c[buf][i]);
      xq::load_scale_bias<B>(srow, brow, gbeg + bi * B, gend, sbv, sb[buf]);
    }
  };
  auto bperm = [](int src_lane, uint32_t v) {
    return uint32_t(__builtin_amdgcn_ds_bpermute(src_lane << 2, int(v)));
  };
  xq::ScaleBias<B> sbr;   // R: the batch's scales and biases of row j
  xq::Codes<BITS> cp[2];  // R: the current pair of groups' codes of row j
  load_batch(0, 0);
  if constexpr (NB > 1) load_batch(1, 1);
  pre();
  const char* src = lds;
  if constexpr (SRC == kSrcStage) {
    xq::stage<NT>(lds, xr, M, 0, G);
  } else if constexpr (SRC == kSrcPlaneLds) {
    xq::dma_plane<NT>(lds, plane, G);
  } else if constexpr (SRC == kSrcBlockLds) {
    xq::dma_plane_block<NT>(lds, plane, G, blocks >> 1);
  } else if constexpr (SRC == kSrcPlane || SRC == kSrcBlockPlane) {
    src = plane;
  }
  const double* qs = reinterpret_cast<const double*>(
      src + (SRC == kSrcBlockLds ? xq::block_q_offset(G) : xq::plane_q_offset(G)));
  const int* es = reinterpret_cast<const int*>(
      src + (SRC == kSrcBlockLds ? xq::block_e_offset(G) : xq::plane_e_offset(G)));
  const int bq = 4 * (blocks >> 1) + kb;  // one-block sources: the lane's activation row
  double acc[2] = {0.0, 0.0}, tot[2] = {0.0, 0.0}, ss[KS > 1 ? SPW : 1][2];
  // A plane read in place: each group's operands are requested PD groups
  // ahead of their use, so the wave waits for memory once, not per group
  // (one block: only that block's operands, and only the wave's own groups,
  // with no copy of the rest into LDS and no barrier before the first group)
  constexpr bool INPLACE = SRC == kSrcPlane || SRC == kSrcBlockPlane;
  constexpr int PD = INPLACE ? (NG < 4 ? NG : 4) : 1;
  struct PlaneOp {
    xq::v4i a0, a1;
    double q0, q1;
    int e0, e1;
  } pf[PD];
  auto load_op = [&](int gl, PlaneOp& o) {
    const int g = min(gbeg + gl, gend - 1);
    if constexpr (SRC == kSrcBlockPlane) {
      const char* ab = src + g * xq::kGroupBytes + (blocks >> 1) * xq::kBlockBytes + lane * 16;
      o.a0 = *reinterpret_cast<const xq::v4i*>(ab);
      o.a1 = o.a0;
      o.q0 = o.q1 = qs[g * 8 + bq];
      o.e0 = o.e1 = es[g * 8 + bq];
    } else {
      const char* ab = src + g * xq::kGroupBytes + lane * 16;
      o.a0 = *reinterpret_cast<const xq::v4i*>(ab);
      o.a1 = *reinterpret_cast<const xq::v4i*>(ab + xq::kBlockBytes);
      o.q0 = qs[g * 8 + kb];
      o.q1 = qs[g * 8 + 4 + kb];
      o.e0 = es[g * 8 + kb];
      o.e1 = es[g * 8 + 4 + kb];
    }
  };
  if constexpr (INPLACE) {
#pragma unroll
    for (int i = 0; i < PD; ++i) load_op(i, pf[i]);
  }
#pragma unroll
  for (int bi = 0; bi < NB; ++bi) {
    const int buf = bi & 1;
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int gl = bi * B + i, g = gbeg + gl;
      if (g < gend) {
        xq::v4i a0, a1;
        double q0 = 0.0, q1 = 0.0;
        int e0 = 1, e1 = 1;
        if constexpr (INPLACE) {
          const PlaneOp& o = pf[gl % PD];
          a0 = o.a0;
          a1 = o.a1;
          q0 = o.q0;
          q1 = o.q1;
          e0 = o.e0;
          e1 = o.e1;
        } else if constexpr (SRC == kSrcBlockLds) {
          // one block: its operand feeds the accumulator of that block
          a0 = *reinterpret_cast<const xq::v4i*>(src + g * xq::kBlockBytes + lane * 16);
          a1 = a0;
          q0 = q1 = qs[g * 8 + bq];
          e0 = e1 = es[g * 8 + bq];
        } else if constexpr (SRC == kSrcReg) {
          a0 = reg_operand(xr, M, 0, g, q0, e0);
          a1 = (blocks & 2) ? reg_operand(xr, M, 1, g, q1, e1) : a0;
          // this lane receives activation row kb of each block: the Q and Eb
          // of that row sit in the lanes that supplied it (l % 16 = 4 kb)
          q0 = __shfl(q0, 4 * kb, 64);
          e0 = __shfl(e0, 4 * kb, 64);
          q1 = __shfl(q1, 4 * kb, 64);
          e1 = __shfl(e1, 4 * kb, 64);
        } else {
          const char* ab = src + g * xq::kGroupBytes + lane * 16;
          a0 = *reinterpret_cast<const xq::v4i*>(ab);
          a1 = *reinterpret_cast<const xq::v4i*>(ab + xq::kBlockBytes);
          q0 = qs[g * 8 + kb];
          q1 = qs[g * 8 + 4 + kb];
          e0 = es[g * 8 + kb];
          e1 = es[g * 8 + 4 + kb];
        }
        xq::Codes<BITS> ci;
        double sc, bs;
        if constexpr (R) {
          if (i == 0) {
#pragma unroll
            for (int w = 0; w < B / 2; ++w) {
              sbr.s[w] = bperm(4 * j + w, rs[buf]);
              sbr.b[w] = bperm(4 * j + w, rb[buf]);
            }
          }
          if constexpr (RG) {
            // group g: the window of row j, k-block kb (lane 4 j + kb)
#pragma unroll
            for (int w = 0; w < xq::Codes<BITS>::W; ++w)
              ci.w[w] = bperm(4 * j + kb, rw[buf][i].w[w]);
          } else if constexpr (BITS == 8) {
            // group g: piece kb of row j (lane 4 j + kb)
            const uint4 r = rc[buf][i];
            const int s0 = 4 * j + kb;
            ci.w[0] = bperm(s0, r.x);
            ci.w[1] = bperm(s0, r.y);
            ci.w[2] = bperm(s0, r.z);
            ci.w[3] = bperm(s0, r.w);
          } else if ((i & 1) == 0) {
            // group g: words 2 kb, 2 kb + 1 of the row's 32 bytes, in piece
            // kb / 2 (lane 4 j + kb / 2); group g + 1 in piece 2 + kb / 2
            const uint4 r = rc[buf][i >> 1];
            const int s0 = 4 * j + (kb >> 1), s1 = s0 + 2;
            const bool odd = kb & 1;
            const uint32_t x0 = bperm(s0, r.x), x1 = bperm(s0, r.y);
            const uint32_t x2 = bperm(s0, r.z), x3 = bperm(s0, r.w);
            const uint32_t y0 = bperm(s1, r.x), y1 = bperm(s1, r.y);
            const uint32_t y2 = bperm(s1, r.z), y3 = bperm(s1, r.w);
            cp[0].w[0] = odd ? x2 : x0;
            cp[0].w[1] = odd ? x3 : x1;
            cp[1].w[0] = odd ? y2 : y0;
            cp[1].w[1] = odd ? y3 : y1;
          }
          if constexpr (BITS == 4) ci = cp[i & 1];
          sc = sbr.scale(i);
          bs = sbr.bias(i);
        } else {
          ci = c[buf][i];
          sc = sb[buf].scale(i);
          bs = sb[buf].bias(i);
        }
        xq::group_step<BITS>(a0, a1, blocks, xq::b_operand<BITS>(ci), q0, q1, e0, e1, sc, bs,
                             acc);
        if constexpr (INPLACE) {
          if (gl + PD < NG) load_op(gl + PD, pf[gl % PD]);
        }
        // a slice ends after its second group, or after the last group of an
        // odd count
        if ((gl & 1) || g + 1 == gend) {
          if constexpr (KS == 1) {
            tot[0] = tot[0] + acc[0];
            tot[1] = tot[1] + acc[1];
          } else {
            ss[gl >> 1][0] = acc[0];
            ss[gl >> 1][1] = acc[1];
          }
          acc[0] = 0.0;
          acc[1] = 0.0;
        }
      }
    }
    if (bi + 2 < NB) load_batch(buf, bi + 2);
  }
  if constexpr (KS == 1) {
    if constexpr (SRC == kSrcStage || SRC == kSrcPlaneLds || SRC == kSrcBlockLds) __syncthreads();
    yt[kb * NC + t * 16 + j] = float(tot[0]);
    yt[(4 + kb) * NC + t * 16 + j] = float(tot[1]);
  } else {
    // slice sums in slice order, from +0, then one rounding to fp32
    if constexpr (SRC == kSrcStage || SRC == kSrcPlaneLds || SRC == kSrcBlockLds) __syncthreads();
    double* red = reinterpret_cast<double*>(lds);
#pragma unroll
    for (int sl = 0; sl < SPW; ++sl) {
      const int gs = ks * SPW + sl;
      if (gs < S) {
        red[((gs * T + t) * 8 + kb) * 16 + j] = ss[sl][0];
        red[((gs * T + t) * 8 + 4 + kb) * 16 + j] = ss[sl][1];
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 8 * NC; i += NT) {
      const int m = i / NC, cc = i - m * NC;
      const int tt = cc >> 4, jj = cc & 15;
      double total = 0.0;
      for (int k = 0; k < S; ++k) total = total + red[((k * T + tt) * 8 + m) * 16 + jj];
      yt[i] = float(total);
    }
  }
  __syncthreads();
}

// Dense projections (modes of ProjEpilogue).  Workgroup tg covers rows
// tg*16T .. tg*16T + 16T - 1 (tile t: rows tg*16T + 16t + j); for kHcUpMix
// (T = 4) it covers columns tg*16 .. tg*16 + 15 of the four streams (tile t:
// rows t*H + tg*16 + j).
template <int BITS, int MODE, int T, int KS, int SPW, int SRC, bool RM = false>
__global__ __launch_bounds__(64 * T * KS) void xq_dense_kernel(QWeight w,
                                                               const uint16_t* __restrict__ x,
                                                               int64_t x_stride, int M,
                                                               const char* __restrict__ plane,
                                                               ProjEpilogue e) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float yt[8 * 16 * T];
  constexpr int NC = 16 * T, NT = 64 * T * KS;
  int tg = blockIdx.x, blk = blockIdx.y;
  if constexpr (SRC == kSrcBlockLds || SRC == kSrcBlockPlane) {
    if (gridDim.y == 1 && gridDim.x % 8 == 0 && e.xcd_blocks) {
      // both four-row blocks, placed by XCD: workgroups are dispatched to
      // the eight XCDs in turn (id mod 8), so XCDs 0-3 take block 0 and 4-7
      // block 1, and each XCD's L2 holds one block of the plane that all its
      // workgroups copy
      const int b = blockIdx.x, xcd = b & 7;
      blk = xcd >> 2;
      tg = (b >> 3) * 4 + (xcd & 3);
      if (tg >= e.xcd_groups) return;  // padding past the last tile (uniform)
    }
  }
  const int j = threadIdx.x & 15, t = (threadIdx.x >> 6) / KS;
  const int n = w.n, G = w.k / xq::kGroup;
  int row, lrow;  // the lane's tile row, and its row-major load row (RM)
  const int jr = (threadIdx.x & 63) >> 2;
  if constexpr (MODE == kHcUpMix) {
    row = t * e.hidden + min(tg * 16 + j, e.hidden - 1);
    lrow = t * e.hidden + min(tg * 16 + jr, e.hidden - 1);
  } else {
    row = min(tg * NC + t * 16 + j, n - 1);
    lrow = min(tg * NC + t * 16 + jr, n - 1);
  }
  RmRows rm;
  if constexpr (RM) {
    rm.codes = w.codes + size_t(lrow) * (size_t(w.k) * BITS / 32);
    rm.scales = w.scales + size_t(lrow) * G;
    rm.biases = w.biases + size_t(lrow) * G;
  }
  ProjFinish<MODE, NC, NT> fin;
  int blocks = M > 4 ? 3 : 1;
  if constexpr (SRC == kSrcBlockLds || SRC == kSrcBlockPlane) {
    // this workgroup's four activation rows: block blk
    blocks = 1 << blk;
    fin.m_lo = 4 * blk;
    fin.m_hi = fin.m_lo + 4;
  }
  fin.begin(e, tg, M, n);
  xq_tiles<BITS, T, KS, SPW, SRC, RM>(w.codes + size_t(row) * (size_t(w.k) * BITS / 32),
                                      w.scales + size_t(row) * G, w.biases + size_t(row) * G,
                                      tiles_sbv<BITS, SPW>(w), w.k, M, blocks,
                                      XRows{x, x_stride}, plane, lds, yt,
                                      [&] { fin.prefetch(e); }, rm);
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

// Copies a plane of G groups (xq_core.hpp layout) into LDS: every thread
// issues all of its loads before its first store.  Ends with a barrier.
// Expert gate/up + SwiGLU for 16 kGuTiles intermediate rows (blockIdx.x) of one plan
// entry and one four-row block of activation rows: with the plane, blockIdx.y
// is an item of the plan (an entry and a block of rows 4b .. 4b + 3 of x that
// holds a member; past the items a workgroup returns at once, so the active
// ones come first in dispatch order); staged, blockIdx.y is the entry and
// blockIdx.z the block of members 4z .. 4z + 3.  Wave (t, p) owns the 16
// intermediate rows of tile t in matrix p (0: gate, 1: up) and streams them
// over the whole depth (load batches kept D deep, so the memory system
// streams while the matrix cores and VALUs work), adding its slice sums in
// slice order from +0.  The up wave leaves its rounded value in LDS; the gate
// wave writes h[row][slot][i] = bf16(bf16(silu(bf16 g)) * bf16 u) for the
// block's member routes (the exact kernels' SwiGLU, moe.hip gate_up_body).
// Operands: the block of the plane of x copied into LDS, or the members
// staged in order.  FULL: the depth is exactly 2 SPW groups and the scales
// and biases load B at a time (the launcher checks their alignment), so the
// group loop is straight-line code whose scheduler overlaps one group's
// operand reads, matrix-core pass and fp64 fold with the next group's.
constexpr int kGuTiles = 2;  // 16-row tiles per gate/up workgroup (2 waves each)

__host__ __device__ constexpr int gate_up_xch_bytes() { return kGuTiles * 64 * 4; }

template <int BITS, int SPW, int SRC, bool FULL>
__global__ __launch_bounds__(128 * kGuTiles) __attribute__((amdgpu_waves_per_eu(4)))
void xq_gate_up_kernel(
    const uint16_t* __restrict__ x, const char* __restrict__ plane,
    const MoePlan* __restrict__ plan, int top_k, QBank gate, QBank up, QWeight sgate, QWeight sup,
    uint16_t* __restrict__ h, int hs) {
  extern __shared__ __align__(16) char lds[];
  __shared__ int ro[8], so[8];
  constexpr int NT = 128 * kGuTiles;
  constexpr int NG = 2 * SPW;                       // groups per wave (at most)
  constexpr int B = tile_batch<BITS, SPW>();
  constexpr int NB = NG / B;                        // load batches per wave
  constexpr int D = NB < 3 ? NB : 3;                // batches in flight
  int entry, blk;
  if constexpr (SRC == kSrcPlaneLds) {
    // blockIdx.y: an item of the plan, (entry, block of rows with a member)
    if (int(blockIdx.y) >= plan->nitems) return;
    const int item = plan->item[blockIdx.y];
    entry = item >> 1;
    blk = item & 1;
  } else {
    entry = blockIdx.y;
    blk = blockIdx.z;
    if (entry >= plan->count || 4 * blk >= plan->m[entry]) return;
  }
  const int M = plan->m[entry];
  const int expert = plan->expert[entry];
  // the entry's member rows and slots, read now (scalar loads that overlap
  // the weight stream) rather than in the epilogue
  const uint32_t* rw32 = reinterpret_cast<const uint32_t*>(plan->row[entry]);
  const uint32_t* sw32 = reinterpret_cast<const uint32_t*>(plan->slot[entry]);
  const uint64_t mrows = uint64_t(rw32[0]) | (uint64_t(rw32[1]) << 32);
  const uint64_t mslots = uint64_t(sw32[0]) | (uint64_t(sw32[1]) << 32);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = wave >> 1, p = wave & 1;
  // the gate and up matrices of an expert have one shape (the launcher checks)
  const QWeight mw = bank_matrix(p ? up : gate, expert, p ? sup : sgate);
  const int inter = mw.n, hidden = mw.k;
  const int i0 = blockIdx.x * 16 * kGuTiles;
  if (i0 >= inter) return;
  const int lane = threadIdx.x & 63, j = lane & 15, kb = lane >> 4;
  const int G = hidden / xq::kGroup;
  const int col = i0 + 16 * t + j;
  const int row = min(col, inter - 1);
  const bool sbv = xq::sb_vector_ok<B>(mw.scales, mw.biases, G);
  const uint32_t* crow = mw.codes + row * (size_t(hidden) * BITS / 32);
  const uint16_t* srow = mw.scales + size_t(row) * G;
  const uint16_t* brow = mw.biases + size_t(row) * G;
  // RM (4-bit, whole batches of 8 groups): the weight stream is read in
  // row-major lane order, lane 4 r + q taking 16 bytes of tile row r (piece q
  // of a pair of groups) and the scale and bias words of groups 2q, 2q + 1 of
  // the batch, so each four adjacent lanes read contiguous bytes of one row;
  // ds_bpermute then gives lane 16 kb + j the matrix-core operand of row j
  // (the words load_codes would have read), so every product is unchanged.
  // 8-bit: one group's 16 bytes per lane (a pure lane permutation); 5 / 6-bit
  // (RMG): lane 4 r + q reads the code window load_codes gives row r and
  // k-block q, and the window's words move to lane 16 q + r
  constexpr bool RMG = (BITS == 5 || BITS == 6) && FULL && B % 2 == 0;
  constexpr bool RM = (BITS == 4 && FULL && B == 8) || (BITS == 8 && FULL && B % 2 == 0) || RMG;
  const int q4 = lane & 3;
  const int lrow = min(i0 + 16 * t + (lane >> 2), inter - 1);
  const uint32_t* lcrow = mw.codes + lrow * (size_t(hidden) * BITS / 32);
  const uint16_t* lsrow = mw.scales + size_t(lrow) * G;
  const uint16_t* lbrow = mw.biases + size_t(lrow) * G;
  xq::Codes<BITS> c[RM ? 1 : D][B];
  xq::ScaleBias<B> sb[RM ? 1 : D];
  constexpr int NP = BITS == 8 ? B : B / 2;  // 16-byte pieces per batch (4 / 8-bit)
  uint4 rc[RM && !RMG ? D : 1][NP > 0 ? NP : 1];
  xq::Codes<BITS> rw[RMG ? D : 1][RMG ? B : 1];
  uint32_t rs[RM ? D : 1], rb[RM ? D : 1];
  auto load_batch = [&](int buf, int bi) {
    const int g0 = bi * B;
    if constexpr (RM) {
      if constexpr (RMG) {
#pragma unroll
        for (int i = 0; i < B; ++i) xq::load_codes<BITS>(lcrow, g0 + i, q4, rw[buf][i]);
      } else {
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) {
          if constexpr (BITS == 8)  // piece q of group g0 + pp
            rc[buf][pp] = *reinterpret_cast<const uint4*>(lcrow + 16 * (g0 + pp) + 4 * q4);
          else  // piece q of groups g0 + 2 pp, + 1
            rc[buf][pp] = *reinterpret_cast<const uint4*>(lcrow + 8 * (g0 + 2 * pp) + 4 * q4);
        }
      }
      // B / 2 scale (bias) words per row; lanes past them repeat the last
      const int qw = q4 & (B / 2 - 1);
      rs[buf] = *reinterpret_cast<const uint32_t*>(lsrow + g0 + 2 * qw);
      rb[buf] = *reinterpret_cast<const uint32_t*>(lbrow + g0 + 2 * qw);
    } else {
#pragma unroll
      for (int i = 0; i < B; ++i) xq::load_codes<BITS>(crow, min(g0 + i, G - 1), kb, c[buf][i]);
      if constexpr (FULL)
        xq::load_scale_bias_vec<B>(srow, brow, g0, sb[buf]);
      else
        xq::load_scale_bias<B>(srow, brow, min(g0, G - 1), G, sbv, sb[buf]);
    }
  };
  auto bperm = [](int src_lane, uint32_t v) {
    return uint32_t(__builtin_amdgcn_ds_bpermute(src_lane << 2, int(v)));
  };
  // operand addresses: group g's A operand at ab + g * gstride; Q and Eb of
  // the lane's activation row at qb[8 g], eb[8 g]
  const char* ab;
  const double* qb;
  const int* eb;
  int gstride, xch_at;
  if constexpr (SRC == kSrcPlaneLds) {
    // the plane block (from the L2) lands first; the weight batches go out
    // after it, so the group loop starts when its first batch arrives rather
    // than after all of them
    xq::dma_plane_block<NT>(lds, plane, G, blk, blockIdx.x + 7 * blockIdx.y);
#pragma unroll
    for (int d = 0; d < D; ++d) load_batch(d, d);
    ab = lds + lane * 16;
    gstride = xq::kBlockBytes;
    qb = reinterpret_cast<const double*>(lds + xq::block_q_offset(G)) + 4 * blk + kb;
    eb = reinterpret_cast<const int*>(lds + xq::block_e_offset(G)) + 4 * blk + kb;
    xch_at = xq::block_bytes(G);
  } else {
    // member rows and slots: loaded before the weights, stored after them,
    // so no wait for them holds the weight loads back
    int r8 = 0, s8 = 0;
    if (threadIdx.x < 8) {
      r8 = plan->row[entry][threadIdx.x];
      s8 = plan->slot[entry][threadIdx.x];
    }
#pragma unroll
    for (int d = 0; d < D; ++d) load_batch(d, d);
    if (threadIdx.x < 8) {
      ro[threadIdx.x] = r8;
      so[threadIdx.x] = s8;
    }
    __syncthreads();
    xq::stage<NT>(lds, MemberRows{x, hidden, 0, ro, so}, M, 0, G);
    ab = lds + blk * xq::kBlockBytes + lane * 16;
    gstride = xq::kGroupBytes;
    qb = reinterpret_cast<const double*>(lds + xq::plane_q_offset(G)) + 4 * blk + kb;
    eb = reinterpret_cast<const int*>(lds + xq::plane_e_offset(G)) + 4 * blk + kb;
    xch_at = xq::stage_bytes(G);
  }
  // the up waves' rounded values: [tile][lane]
  float* xch = reinterpret_cast<float*>(lds + ((xch_at + 15) & ~15));
  double tot = 0.0, acc = 0.0;
  xq::ScaleBias<B> sbr;   // RM: the batch's scales and biases of row j
  xq::Codes<BITS> cp[2];  // RM: the current pair of groups' codes of row j
#pragma unroll
  for (int bi = 0; bi < NB; ++bi) {
    const int buf = bi % D;
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int gl = bi * B + i;
      if (FULL || gl < G) {
        xq::Codes<BITS> ci;
        double sc, bs;
        if constexpr (RM) {
          if (i == 0) {
#pragma unroll
            for (int w = 0; w < B / 2; ++w) {
              sbr.s[w] = bperm(4 * j + w, rs[buf]);
              sbr.b[w] = bperm(4 * j + w, rb[buf]);
            }
          }
          if constexpr (RMG) {
            // group gl: the window of row j, k-block kb (lane 4 j + kb)
#pragma unroll
            for (int w = 0; w < xq::Codes<BITS>::W; ++w)
              ci.w[w] = bperm(4 * j + kb, rw[buf][i].w[w]);
          } else if constexpr (BITS == 8) {
            // group gl: piece kb of row j (lane 4 j + kb)
            const uint4 r = rc[buf][i];
            const int s0 = 4 * j + kb;
            ci.w[0] = bperm(s0, r.x);
            ci.w[1] = bperm(s0, r.y);
            ci.w[2] = bperm(s0, r.z);
            ci.w[3] = bperm(s0, r.w);
          } else if ((i & 1) == 0) {
            // group gl: words 2 kb, 2 kb + 1 of the row's 32 bytes, in piece
            // kb / 2 (lane 4 j + kb / 2); group gl + 1 in piece 2 + kb / 2
            const uint4 r = rc[buf][i >> 1];
            const int s0 = 4 * j + (kb >> 1), s1 = s0 + 2;
            const bool odd = kb & 1;
            const uint32_t a0 = bperm(s0, r.x), a1 = bperm(s0, r.y);
            const uint32_t a2 = bperm(s0, r.z), a3 = bperm(s0, r.w);
            const uint32_t b0 = bperm(s1, r.x), b1 = bperm(s1, r.y);
            const uint32_t b2 = bperm(s1, r.z), b3 = bperm(s1, r.w);
            cp[0].w[0] = odd ? a2 : a0;
            cp[0].w[1] = odd ? a3 : a1;
            cp[1].w[0] = odd ? b2 : b0;
            cp[1].w[1] = odd ? b3 : b1;
          }
          if constexpr (BITS == 4) ci = cp[i & 1];
          sc = sbr.scale(i);
          bs = sbr.bias(i);
        } else {
          ci = c[buf][i];
          sc = sb[buf].scale(i);
          bs = sb[buf].bias(i);
        }
        xq::group_step1<BITS>(*reinterpret_cast<const xq::v4i*>(ab + gl * gstride),
                              xq::b_operand<BITS>(ci), qb[gl * 8], eb[gl * 8], sc, bs, acc);
        // a slice ends after its second group, or after the last of an odd count
        // (no scheduling barrier here: letting the compiler interleave the
        // groups of neighbouring slices measured 25.2 against 27.0 us)
        if ((gl & 1) || (!FULL && gl + 1 == G)) {
          tot = tot + acc;
          acc = 0.0;
        }
      }
    }
    if (bi + D < NB) load_batch(buf, bi + D);
  }
  const float v = round_bf16(float(tot));
  if (p) xch[t * 64 + lane] = v;
  __syncthreads();
  if (p) return;
  // lane (kb, j) holds activation row (plane) or member (staged) 4 blk + kb
  // of column col
  const int xr = 4 * blk + kb;
  if (col < inter) {
    const float uv = xch[t * 64 + lane];
    const float silu = round_bf16(v * sigmoid_bf16(v));
    const uint16_t out = f32_to_bf16(silu * uv);
    for (int m = 0; m < M; ++m) {
      if constexpr (SRC == kSrcPlaneLds) {
        const int r = int((mrows >> (8 * m)) & 0xffu);
        if (r == xr) h[(size_t(r) * (top_k + 1) + int((mslots >> (8 * m)) & 0xffu)) * hs + col] = out;
      } else {
        if (m == xr) h[(size_t(ro[m]) * (top_k + 1) + so[m]) * hs + col] = out;
      }
    }
  }
}

constexpr int kDnTiles = 4;  // 16-column tiles per expert down workgroup (one wave each)

// Expert down + route score for one plan entry (blockIdx.y) and 16 kDnTiles output
// columns (blockIdx.x): p[row][slot][c] = bf16(bf16(down h) * score) for
// routed slots, bf16(down h) for the shared slot (moe.hip down_body).
template <int BITS, int SPW>
__global__ __launch_bounds__(64 * kDnTiles) void xq_down_kernel(const uint16_t* __restrict__ h,
                                                      const MoePlan* __restrict__ plan,
                                                      const uint16_t* __restrict__ scores,
                                                      int top_k, QBank down, QWeight sdown,
                                                      uint16_t* __restrict__ p, int hs) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float yt[8 * 16 * kDnTiles];
  __shared__ int ro[8], so[8];
  __shared__ float sco[8];
  const int entry = blockIdx.y;
  if (entry >= plan->count) return;
  const int expert = plan->expert[entry];
  const QWeight dw = bank_matrix(down, expert, sdown);
  const int hidden = dw.n, inter = dw.k;
  const int c0 = blockIdx.x * 16 * kDnTiles;
  if (c0 >= hidden) return;
  const int M = plan->m[entry];
  if (threadIdx.x < 8) {
    // member rows, slots and route scores (the epilogue's), read up front
    const int r = plan->row[entry][threadIdx.x], sl = plan->slot[entry][threadIdx.x];
    ro[threadIdx.x] = r;
    so[threadIdx.x] = sl;
    sco[threadIdx.x] = int(threadIdx.x) < M && sl < top_k
                           ? bf16_to_f32(scores[size_t(r) * top_k + sl])
                           : 1.0f;
  }
  __syncthreads();
  const int j = threadIdx.x & 15, t = threadIdx.x >> 6;
  const int row = min(c0 + 16 * t + j, hidden - 1);
  const int G = inter / xq::kGroup;
  xq_tiles<BITS, kDnTiles, 1, SPW, kSrcStage>(dw.codes + size_t(row) * (size_t(inter) * BITS / 32),
                                       dw.scales + size_t(row) * G, dw.biases + size_t(row) * G,
                                       tiles_sbv<BITS, SPW>(dw), inter, M, M > 4 ? 3 : 1,
                                       MemberRows{h, int64_t(top_k + 1) * hs, hs, ro, so}, nullptr,
                                       lds, yt, [] {});
  constexpr int NC = 16 * kDnTiles;
  for (int i = threadIdx.x; i < 8 * NC; i += 64 * kDnTiles) {
    const int m = i / NC, c = i % NC;
    if (m >= M || c0 + c >= hidden) continue;
    const bool routed = so[m] < top_k;
    const float dv = round_bf16(yt[i]);
    p[(size_t(ro[m]) * (top_k + 1) + so[m]) * hidden + c0 + c] =
        f32_to_bf16(routed ? dv * sco[m] : dv);
  }
}

// Hyper-connection up-projection and stream mix for one 64-column group of
// `mixed` (blockIdx.x = tg) and, with more than four activation rows, one
// four-row block of them (blockIdx.y): tile t = 4 s + ct holds up rows
// s * H + 64 tg + 16 ct + j (K = the rank); each column takes the kHcUpMix
// arithmetic of ProjFinish, then wave 0 writes the group's operand plane, so
// every consumer of `mixed` reads its operands ready-made.
template <int BITS, int SPW, bool RM = false>
__global__ __launch_bounds__(1024) void xq_upmix_kernel(QWeight w, const uint16_t* __restrict__ lo,
                                                        int M, const uint16_t* __restrict__ xn,
                                                        int hidden, uint16_t* __restrict__ mixed,
                                                        char* __restrict__ plane) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float yt[8 * 256];
  __shared__ float mix[8 * 64];
  const int tg = blockIdx.x;
  const int j = threadIdx.x & 15, t = threadIdx.x >> 6;
  const int row = (t >> 2) * hidden + tg * 64 + (t & 3) * 16 + j;
  const int G = w.k / xq::kGroup;
  RmRows rm;
  if constexpr (RM) {
    // the lane's row-major load row: tile row (lane & 63) / 4
    const int lrow = (t >> 2) * hidden + tg * 64 + (t & 3) * 16 + ((threadIdx.x & 63) >> 2);
    rm.codes = w.codes + size_t(lrow) * (size_t(w.k) * BITS / 32);
    rm.scales = w.scales + size_t(lrow) * G;
    rm.biases = w.biases + size_t(lrow) * G;
  }
  // two workgroups per column group when there are two four-row blocks of
  // activation rows: blockIdx.y = the block this one computes and writes
  const bool split = gridDim.y > 1;
  const int mlo = split ? 4 * int(blockIdx.y) : 0, mhi = split ? mlo + 4 : 8;
  // the normed streams the mix multiplies, requested once the first weight
  // loads are out (thread i < 512 mixes row i / 64, column i % 64)
  const int im = threadIdx.x >> 6, ic = threadIdx.x & 63;
  const bool mixer = threadIdx.x < 8 * 64 && im < M && im >= mlo && im < mhi;
  uint16_t xv[4] = {0, 0, 0, 0};
  xq_tiles<BITS, 16, 1, SPW, kSrcStage, RM>(
      w.codes + size_t(row) * (size_t(w.k) * BITS / 32), w.scales + size_t(row) * G,
      w.biases + size_t(row) * G, tiles_sbv<BITS, SPW>(w), w.k, M,
      split ? 1 << blockIdx.y : (M > 4 ? 3 : 1), XRows{lo, w.k}, nullptr, lds, yt,
      [&] {
        if (mixer) {
#pragma unroll
          for (int s = 0; s < 4; ++s)
            xv[s] = xn[size_t(im) * 4 * hidden + size_t(s) * hidden + tg * 64 + ic];
        }
      },
      rm);
  for (int i = threadIdx.x; i < 8 * 64; i += 1024) {
    const int m = i >> 6, c = i & 63;
    float v = 0.0f;
    if (m < M && m >= mlo && m < mhi) {
      float sum = 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float p = round_bf16(yt[m * 256 + s * 64 + c]);
        const float x = bf16_to_f32(xv[s]);
        sum = sum + round_bf16(sigmoid_bf16(p) * x);
      }
      const uint16_t o = f32_to_bf16(round_bf16(sum) / 4.0f);
      mixed[size_t(m) * hidden + tg * 64 + c] = o;
      v = bf16_to_f32(o);
    }
    mix[i] = v;
  }
  if (!plane) return;
  __syncthreads();
  if (threadIdx.x < 64) {
    // lane l: row l % 8 (lanes with l % 16 >= 8 repeat a row and only join
    // the butterflies), values 16 (l / 16) .. +15 of the group
    const int lane = threadIdx.x, m = lane & 7, kb = lane >> 4;
    float f[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = mix[m * 64 + 16 * kb + i];
    xq::digitize_unit(f, m, tg, kb, (lane & 15) < 8 && m < M && m >= mlo && m < mhi, plane,
                      hidden / xq::kGroup);
  }
}

__device__ __forceinline__ void better_of(float v, uint32_t id, float& best, uint32_t& best_id) {
  if (v > best || (v == best && id < best_id)) {
    best = v;
    best_id = id;
  }
}

// Greedy head: per activation row, the best (bf16 logit, lowest id) of the
// workgroup's 256 vocabulary rows (16 waves, each streaming a 16-row tile
// over the whole depth; NaN never wins; nothing above -inf keeps id
// 0xffffffff), and, when asked, the bf16 logits themselves.
template <int BITS, int SPW, int SRC, bool RM = false>
__global__ __launch_bounds__(1024) void xq_head_kernel(QWeight w, const uint16_t* __restrict__ x,
                                                       const char* __restrict__ plane, int M,
                                                       float* __restrict__ maxima,
                                                       uint32_t* __restrict__ indices,
                                                       uint16_t* __restrict__ logits) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float yt[8 * 256];
  __shared__ float bv[16][8];
  __shared__ uint32_t bi[16][8];
  const int tg = blockIdx.x, parts = gridDim.x;
  const int j = threadIdx.x & 15, t = threadIdx.x >> 6;
  const int n = w.n, G = w.k / xq::kGroup;
  const int row = min(tg * 256 + 16 * t + j, n - 1);
  RmRows rm;
  if constexpr (RM) {
    // the lane's row-major load row: tile row (lane & 63) / 4
    const int lrow = min(tg * 256 + 16 * t + ((threadIdx.x & 63) >> 2), n - 1);
    rm.codes = w.codes + size_t(lrow) * (size_t(w.k) * BITS / 32);
    rm.scales = w.scales + size_t(lrow) * G;
    rm.biases = w.biases + size_t(lrow) * G;
  }
  xq_tiles<BITS, 16, 1, SPW, SRC, RM>(w.codes + size_t(row) * (size_t(w.k) * BITS / 32),
                                      w.scales + size_t(row) * G, w.biases + size_t(row) * G,
                                      tiles_sbv<BITS, SPW>(w), w.k, M, M > 4 ? 3 : 1,
                                      XRows{x, w.k}, plane, lds, yt, [] {}, rm);
  // wave t ranks columns 16 t .. +15 for every row (lane = 16 m' + c, two
  // passes of four rows), then wave 0 ranks the 16 wave bests per row
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int m = 4 * half + (lane >> 4), c = 16 * t + (lane & 15);
    const int r = tg * 256 + c;
    float best = u2f(0xff800000u);
    uint32_t best_id = 0xffffffffu;
    if (m < M && r < n) {
      better_of(round_bf16(yt[m * 256 + c]), uint32_t(r), best, best_id);
      if (logits) logits[size_t(m) * n + r] = f32_to_bf16(yt[m * 256 + c]);
    }
    for (int o = 8; o > 0; o >>= 1) {
      const float v = __shfl_xor(best, o, 64);
      const uint32_t id = uint32_t(__shfl_xor(int(best_id), o, 64));
      better_of(v, id, best, best_id);
    }
    if ((lane & 15) == 0) {
      bv[t][m] = best;
      bi[t][m] = best_id;
    }
  }
  __syncthreads();
  if (threadIdx.x < 8 && int(threadIdx.x) < M) {
    const int m = threadIdx.x;
    float best = bv[0][m];
    uint32_t best_id = bi[0][m];
    for (int w2 = 1; w2 < 16; ++w2) better_of(bv[w2][m], bi[w2][m], best, best_id);
    maxima[size_t(m) * parts + tg] = best;
    indices[size_t(m) * parts + tg] = best_id;
  }
}

template <int BITS, int MODE, int T, int KS, int SPW, int SRC>
int launch_xq(const QWeight& w, const uint16_t* x, int64_t xs, int m, const char* plane,
              const ProjEpilogue& e, hipStream_t s) {
  const int groups = MODE == kHcUpMix ? (e.hidden + 15) / 16 : (w.n + 16 * T - 1) / (16 * T);
  const int lb = tiles_lds(w.k / xq::kGroup, T, KS, SRC);
  auto fn = xq_dense_kernel<BITS, MODE, T, KS, SPW, SRC, false>;
  constexpr int B = tile_batch<BITS, SPW>();
  if constexpr (B % 2 == 0) {
    // row-major weight reads: the KS waves of a tile cover the depth in whole
    // batches (no wave reads past its row), rows on 16-byte boundaries, the
    // scale/bias rows aligned for B-group reads
    const int G = w.k / xq::kGroup;
    const bool rm = G == KS * 2 * SPW &&
                    (BITS == 5 || BITS == 6 ||
                     ((reinterpret_cast<uintptr_t>(w.codes) & 15) == 0 &&
                      (size_t(w.k) * BITS / 8) % 16 == 0)) &&
                    xq::sb_vector_ok<B>(w.scales, w.biases, G);
    if (rm) fn = xq_dense_kernel<BITS, MODE, T, KS, SPW, SRC, true>;
  }
  MX_TRY_RC(raise_lds(fn, lb));
  const int nblk = (SRC == kSrcBlockLds || SRC == kSrcBlockPlane) && m > 4 ? 2 : 1;
  if (nblk == 2) {
    // one-dimensional grid placed by XCD (xq_dense_kernel)
    ProjEpilogue ex = e;
    ex.xcd_blocks = 1;
    ex.xcd_groups = groups;
    hipLaunchKernelGGL(fn, dim3((groups + 3) / 4 * 8, 1), dim3(64 * T * KS), lb, s, w, x, xs, m,
                       plane, ex);
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
  }
  hipLaunchKernelGGL(fn, dim3(groups, nblk), dim3(64 * T * KS), lb, s, w, x, xs, m, plane, e);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

// Slices of two groups: S = 1..4 slices run in one wave (four tiles per
// workgroup); deeper rows split their slices over KS waves of one tile (16
// waves at K = 2048 for up to 2048 rows, so short matrices still fill the
// chip) or of four tiles (long matrices).  Operands come from the caller's
// plane when there is one (read in place by one-tile shapes, copied to LDS
// by four-tile ones), else from an LDS staging (up to 64 groups) or from
// registers.
template <int BITS, int MODE>
int xq_shape(const QWeight& w, const uint16_t* x, int64_t xs, int m, const char* plane,
             const ProjEpilogue& e, hipStream_t s) {
  const int G = w.k / xq::kGroup, S = (G + 1) / 2;
#define MX_XQ(T_, KS_, SPW_, SRC_) \
  return launch_xq<BITS, MODE, T_, KS_, SPW_, SRC_>(w, x, xs, m, plane, e, s)
  if (S <= 4) {
    if (S == 1) MX_XQ(4, 1, 1, kSrcStage);
    if (S == 2) MX_XQ(4, 1, 2, kSrcStage);
    MX_XQ(4, 1, 4, kSrcStage);
  }
  if constexpr (MODE != kHcUpMix) {
    if (S == 8) {
      if (plane) MX_XQ(4, 2, 4, kSrcPlaneLds);
      MX_XQ(4, 2, 4, kSrcStage);
    }
    if (S == 16) {
      if (w.n > 2048) {
        if (plane) MX_XQ(4, 4, 4, kSrcPlaneLds);
        MX_XQ(4, 4, 4, kSrcStage);
      }
      if (plane) MX_XQ(1, 16, 1, kSrcPlane);
      MX_XQ(1, 16, 1, kSrcStage);
    }
    if (S == 32) {
      if (plane) MX_XQ(1, 16, 2, kSrcPlane);
      MX_XQ(1, 8, 4, kSrcStage);
    }
    if (S == 64) {
      // each workgroup takes one block of the plane; each wave reads its own
      // groups' operands of that block in place
      if (plane) MX_XQ(1, 16, 4, kSrcBlockPlane);
      MX_XQ(1, 16, 4, kSrcReg);
    }
  }
#undef MX_XQ
  return MX_EUNSUPPORTED;
}

template <int BITS>
int xq_mode(const QWeight& w, const uint16_t* x, int64_t xs, int m, const char* plane,
            const ProjEpilogue& e, hipStream_t s) {
  switch (e.mode) {
    case kPlain: return xq_shape<BITS, kPlain>(w, x, xs, m, plane, e, s);
    case kHcDown: return xq_shape<BITS, kHcDown>(w, x, xs, m, plane, e, s);
    case kHcUpMix: return xq_shape<BITS, kHcUpMix>(w, x, xs, m, plane, e, s);
    case kConv:
      if constexpr (BITS == 4) return xq_shape<BITS, kConv>(w, x, xs, m, plane, e, s);
      return MX_EUNSUPPORTED;
    default: return xq_shape<BITS, kHcWrite>(w, x, xs, m, plane, e, s);
  }
}

// Slices per wave of a whole-depth shape: S rounded up to a power of two.
int whole_spw(int k) {
  const int S = (k / xq::kGroup + 1) / 2;
  int spw = 1;
  while (spw < S) spw *= 2;
  return spw;
}

template <int BITS, int SPW>
int launch_gate_up(const uint16_t* x, const char* plane, const MoePlan* plan, int routes,
                   int top_k, const QBank& gate, const QBank& up, const QWeight& sgate,
                   const QWeight& sup, uint16_t* h, int hs, hipStream_t s) {
  const int gx = (hs + 16 * kGuTiles - 1) / (16 * kGuTiles);
  // plane: one workgroup row per plan item (an entry's items are the blocks
  // its routes come from, so there are at most routes + 1 of them: the shared
  // entry's two blocks and at most one per routed route); staged: entries by
  // blocks of members
  const dim3 grid = plane ? dim3(gx, routes + 1, 1) : dim3(gx, routes, 2);
  const int G = gate.k / xq::kGroup;
  const int lb = ((plane ? xq::block_bytes(G) : xq::stage_bytes(G)) + 15) / 16 * 16 +
                 gate_up_xch_bytes();
  // FULL also needs every expert's scale/bias rows on 2B-byte boundaries
  constexpr int B = tile_batch<BITS, SPW>();
  const bool full = G == 2 * SPW && xq::sb_vector_ok<B>(gate.scales, gate.biases, G) &&
                    xq::sb_vector_ok<B>(up.scales, up.biases, G) &&
                    xq::sb_vector_ok<B>(sgate.scales, sgate.biases, G) &&
                    xq::sb_vector_ok<B>(sup.scales, sup.biases, G) &&
                    (size_t(gate.n) * G) % B == 0 && (size_t(up.n) * G) % B == 0 &&
                    // FULL 4- and 8-bit forms read 16-byte code pieces
                    ((reinterpret_cast<uintptr_t>(gate.codes) | reinterpret_cast<uintptr_t>(up.codes) |
                      reinterpret_cast<uintptr_t>(sgate.codes) | reinterpret_cast<uintptr_t>(sup.codes)) &
                     15) == 0;
  const auto fn = plane ? (full ? xq_gate_up_kernel<BITS, SPW, kSrcPlaneLds, true>
                                : xq_gate_up_kernel<BITS, SPW, kSrcPlaneLds, false>)
                        : (full ? xq_gate_up_kernel<BITS, SPW, kSrcStage, true>
                                : xq_gate_up_kernel<BITS, SPW, kSrcStage, false>);
  MX_TRY_RC(raise_lds(fn, lb));
  hipLaunchKernelGGL(fn, grid, dim3(128 * kGuTiles), lb, s, x, plane, plan, top_k, gate, up,
                     sgate, sup, h, hs);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

template <int BITS, int SPW>
int launch_down(const uint16_t* h, const MoePlan* plan, int routes, const uint16_t* scores,
                int top_k, const QBank& down, const QWeight& sdown, uint16_t* p, int hs,
                hipStream_t s) {
  const auto fn = xq_down_kernel<BITS, SPW>;
  const int kmax = down.k > sdown.k ? down.k : sdown.k;
  const int lb = tiles_lds(kmax / xq::kGroup, kDnTiles, 1, kSrcStage);
  MX_TRY_RC(raise_lds(fn, lb));
  constexpr int NC = 16 * kDnTiles;
  hipLaunchKernelGGL(fn, dim3((down.n + NC - 1) / NC, routes), dim3(64 * kDnTiles), lb, s, h,
                     plan, scores, top_k, down, sdown, p, hs);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

template <int BITS, int SPW>
int launch_head(const QWeight& w, const uint16_t* x, const char* plane, int m, float* maxima,
                uint32_t* indices, uint16_t* logits, int parts, hipStream_t s) {
  const int G = w.k / xq::kGroup;
  constexpr int B = tile_batch<BITS, SPW>();
  // row-major weight reads (8-bit; 4-bit with even batches): whole batches
  // over the depth, rows on 16-byte boundaries, scale/bias rows aligned
  const bool rm = (BITS == 8 || (BITS == 4 && B % 2 == 0)) && G == 2 * SPW &&
                  (reinterpret_cast<uintptr_t>(w.codes) & 15) == 0 &&
                  (size_t(w.k) * BITS / 8) % 16 == 0 && B > 1 &&
                  xq::sb_vector_ok<(B > 1 ? B : 2)>(w.scales, w.biases, G);
  if (plane && rm && (BITS == 8 || BITS == 4)) {
    const auto fn = xq_head_kernel<BITS, SPW, kSrcPlaneLds, BITS == 8 || BITS == 4>;
    const int lb = tiles_lds(G, 16, 1, kSrcPlaneLds);
    MX_TRY_RC(raise_lds(fn, lb));
    hipLaunchKernelGGL(fn, dim3(parts), dim3(1024), lb, s, w, x, plane, m, maxima, indices, logits);
  } else if (plane) {
    const auto fn = xq_head_kernel<BITS, SPW, kSrcPlaneLds>;
    const int lb = tiles_lds(G, 16, 1, kSrcPlaneLds);
    MX_TRY_RC(raise_lds(fn, lb));
    hipLaunchKernelGGL(fn, dim3(parts), dim3(1024), lb, s, w, x, plane, m, maxima, indices, logits);
  } else {
    const auto fn = xq_head_kernel<BITS, SPW, kSrcStage>;
    const int lb = tiles_lds(G, 16, 1, kSrcStage);
    MX_TRY_RC(raise_lds(fn, lb));
    hipLaunchKernelGGL(fn, dim3(parts), dim3(1024), lb, s, w, x, plane, m, maxima, indices, logits);
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

// Expert and head matrices: K a multiple of 64 up to 2048 (one whole-depth
// wave per tile, operands staged or copied into LDS).
bool xq_whole_ok(int k) { return k % 64 == 0 && k >= 64 && k <= 2048; }

#define MX_SPW_DISPATCH(B_, FN, ...)                          \
  switch (spw) {                                              \
    case 1: return FN<B_, 1>(__VA_ARGS__);                    \
    case 2: return FN<B_, 2>(__VA_ARGS__);                    \
    case 4: return FN<B_, 4>(__VA_ARGS__);                    \
    case 8: return FN<B_, 8>(__VA_ARGS__);                    \
    default: return FN<B_, 16>(__VA_ARGS__);                  \
  }

}  // namespace

int xq_gate_up(const uint16_t* x, const char* plane, const MoePlan* plan, int rows, int top_k,
               const QBank& gate, const QBank& up, const QWeight& sgate, const QWeight& sup,
               uint16_t* h, hipStream_t s) {
  if (gate.group_size != 64 || up.group_size != 64 || sgate.group_size != 64 ||
      sup.group_size != 64 || !xq_whole_ok(gate.k) || sgate.k != gate.k || up.k != gate.k ||
      gate.bits != up.bits || sgate.bits != gate.bits || sup.bits != gate.bits ||
      up.n != gate.n || sup.n != sgate.n)
    return MX_EUNSUPPORTED;
  const int routes = rows * top_k + 1;
  const int hs = gate.n > sgate.n ? gate.n : sgate.n;
  // two waves per tile (gate and up), each over the whole depth
  const int spw = whole_spw(gate.k);
  switch (gate.bits) {
    case 4: MX_SPW_DISPATCH(4, launch_gate_up, x, plane, plan, routes, top_k, gate, up, sgate, sup, h, hs, s)
    case 5: MX_SPW_DISPATCH(5, launch_gate_up, x, plane, plan, routes, top_k, gate, up, sgate, sup, h, hs, s)
    case 6: MX_SPW_DISPATCH(6, launch_gate_up, x, plane, plan, routes, top_k, gate, up, sgate, sup, h, hs, s)
    default: MX_SPW_DISPATCH(8, launch_gate_up, x, plane, plan, routes, top_k, gate, up, sgate, sup, h, hs, s)
  }
}

int xq_down(const uint16_t* h, const MoePlan* plan, const uint16_t* scores, int rows, int top_k,
            int inter, int shared_inter, const QBank& down, const QWeight& sdown, uint16_t* p,
            hipStream_t s) {
  if (down.group_size != 64 || sdown.group_size != 64 || !xq_whole_ok(down.k) ||
      !xq_whole_ok(sdown.k) || sdown.bits != down.bits || sdown.n != down.n)
    return MX_EUNSUPPORTED;
  const int routes = rows * top_k + 1;
  const int hs = inter > shared_inter ? inter : shared_inter;
  const int spw = whole_spw(down.k > sdown.k ? down.k : sdown.k);
  switch (down.bits) {
    case 4: MX_SPW_DISPATCH(4, launch_down, h, plan, routes, scores, top_k, down, sdown, p, hs, s)
    case 5: MX_SPW_DISPATCH(5, launch_down, h, plan, routes, scores, top_k, down, sdown, p, hs, s)
    case 6: MX_SPW_DISPATCH(6, launch_down, h, plan, routes, scores, top_k, down, sdown, p, hs, s)
    default: MX_SPW_DISPATCH(8, launch_down, h, plan, routes, scores, top_k, down, sdown, p, hs, s)
  }
}

int xq_upmix(const QWeight& up, const uint16_t* lo, int m, const uint16_t* xn, int hidden,
             uint16_t* mixed, char* mixed_plane, hipStream_t s) {
  if (up.group_size != 64 || up.k % 64 != 0 || up.k > 512 || up.n != 4 * hidden ||
      hidden % 64 != 0 || m < 1 || m > 8)
    return MX_EUNSUPPORTED;
  const int G = up.k / xq::kGroup;
  const int lb = tiles_lds(G, 16, 1, kSrcStage);
  const dim3 grid(hidden / 64, m > 4 ? 2 : 1);
  const int spw = whole_spw(up.k);
  // row-major weight reads (4-bit): the tile's waves cover the depth in whole
  // batches, rows on 16-byte boundaries, scale/bias rows aligned
  const bool rm = up.bits == 4 && G == 2 * spw && (reinterpret_cast<uintptr_t>(up.codes) & 15) == 0 &&
                  (size_t(up.k) * 4 / 8) % 16 == 0;
#define MX_UM(B, SPW)                                                                           \
  if (up.bits == B && spw == SPW) {                                                             \
    if (B == 4 && rm &&                                                                         \
        xq::sb_vector_ok<tile_batch<B, SPW>()>(up.scales, up.biases, G))                         \
      hipLaunchKernelGGL((xq_upmix_kernel<B, SPW, B == 4>), grid, dim3(1024), lb, s, up, lo, m,  \
                         xn, hidden, mixed, mixed_plane);                                       \
    else                                                                                        \
      hipLaunchKernelGGL((xq_upmix_kernel<B, SPW, false>), grid, dim3(1024), lb, s, up, lo, m,   \
                         xn, hidden, mixed, mixed_plane);                                       \
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;                                   \
  }
  MX_UM(4, 1) MX_UM(4, 2) MX_UM(4, 4) MX_UM(5, 1) MX_UM(5, 2) MX_UM(5, 4)
  MX_UM(6, 1) MX_UM(6, 2) MX_UM(6, 4) MX_UM(8, 1) MX_UM(8, 2) MX_UM(8, 4)
#undef MX_UM
  return MX_EUNSUPPORTED;
}

size_t xq_plane_bytes(int k) { return size_t(xq::stage_bytes(k / xq::kGroup)); }

int xq_head_parts(int n) { return (n + 255) / 256; }

int xq_head(const QWeight& w, const uint16_t* x, const char* plane, int m, float* maxima,
            uint32_t* indices, uint16_t* logits, int* parts_out, hipStream_t s) {
  if (w.group_size != 64 || !xq_whole_ok(w.k) || m < 1 || m > 8) return MX_EUNSUPPORTED;
  const int parts = xq_head_parts(w.n);
  *parts_out = parts;
  const int spw = whole_spw(w.k);
  switch (w.bits) {
    case 4: MX_SPW_DISPATCH(4, launch_head, w, x, plane, m, maxima, indices, logits, parts, s)
    case 5: MX_SPW_DISPATCH(5, launch_head, w, x, plane, m, maxima, indices, logits, parts, s)
    case 6: MX_SPW_DISPATCH(6, launch_head, w, x, plane, m, maxima, indices, logits, parts, s)
    default: MX_SPW_DISPATCH(8, launch_head, w, x, plane, m, maxima, indices, logits, parts, s)
  }
}

// Group size 64; K a multiple of 64 with at most four slices (K <= 512), or
// K = 1024, 2048, 4096 or 8192.
bool xq_supported(const QWeight& w) {
  const bool shape = w.k % 64 == 0 && w.k >= 64 &&
                     (w.k <= 512 || w.k == 1024 || w.k == 2048 || w.k == 4096 || w.k == 8192);
  return w.group_size == 64 && shape && (w.bits == 4 || w.bits == 5 || w.bits == 6 || w.bits == 8);
}

int xq_dense(const QWeight& w, const uint16_t* x, int64_t x_stride, int m, const ProjEpilogue& e,
             hipStream_t s, const char* plane) {
  if (!xq_supported(w) || m < 1 || m > 8) return MX_EUNSUPPORTED;
  if (e.mode == kHcUpMix && e.hidden * 4 != w.n) return MX_EUNSUPPORTED;
  if (e.mode == kConv && (e.taps < 2 || e.taps > kConvMaxTaps)) return MX_EUNSUPPORTED;
  switch (w.bits) {
    case 4: return xq_mode<4>(w, x, x_stride, m, plane, e, s);
    case 5: return xq_mode<5>(w, x, x_stride, m, plane, e, s);
    case 6: return xq_mode<6>(w, x, x_stride, m, plane, e, s);
    default: return xq_mode<8>(w, x, x_stride, m, plane, e, s);
  }
}

}  // namespace mx
