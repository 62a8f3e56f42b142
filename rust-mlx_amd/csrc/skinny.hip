// Decode projections on the gfx950 matrix cores for 1..8 activation rows
// (the arithmetic of skinny_core.hpp): dense projections with the engine's
// fused epilogues, the gathered expert gate/up (+SwiGLU) and down (+route
// score), and the greedy vocabulary head (argmax partials).
//
// Replaces the same reference interfaces as the exact kernels: the QMV /
// gather_qmm rows of Linear::forward_rows (src/weights.rs:111-202,
// src/qmv_kernel.rs:49-180), the expert gather_qmm of MoE::parts
// (src/hybrid.rs:245-271, moe_kernel::gate_up src/moe_kernel.rs:10-118,
// moe_down::reduce src/moe_down.rs:34-137) and greedy_head::project
// (src/greedy_head.rs:40-126).  Results agree with the exact kernels up to
// fp32 summation order, not bit for bit.
//
// A workgroup holds T tiles of 16 weight rows and splits K among KS waves per
// tile (T * KS <= 16 waves); the KS partial sums of a tile are added in slice
// order through LDS, so results are deterministic and no workgroup waits on
// another.  Matrices with few rows use many slices to fill the chip.  For
// K <= 2048 the activation rows are staged once per workgroup in LDS; deeper
// rows are read by each wave straight into registers (group sums of x are
// always staged).  Every wave issues its first weight loads before the
// staging, so the two latencies overlap.
#include "common.hpp"
#include "kernels.hpp"
#include "skinny_core.hpp"
#include "route_core.hpp"
#include "proj_epilogue.hpp"

namespace mx {

namespace {

using sk::floatx4_t;

// Largest K staged in LDS (super-steps); deeper rows stream x into registers,
// up to kDenseSteps.  Expert down rows are at most kDownSteps deep.
constexpr int kStageSteps = 16;
constexpr int kDenseSteps = 64;
constexpr int kDownSteps = 8;
// Waves per gate/up tile (K split inside the workgroup): halves each wave's
// registers so more workgroups stay resident.
constexpr int kGateUpSplit = 2;
// persistent gate/up: 16-row tiles per item and waves per tile (depth split)
constexpr int kPersistTiles = 4;
constexpr int kPersistSplit = 2;

// Sums the KS slices of each tile into yt[m][t * 16 + j] (fp32 [8][16 T]).
// red: LDS [KS][T][8][16] (unused when KS == 1).  Ends with a barrier.
template <int T, int KS>
__device__ __forceinline__ void reduce_tiles(float (&y)[4], float* red, float* yt) {
  sk::join_parities(y);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  const int t = wave / KS, ks = wave - t * KS;
  constexpr int NC = 16 * T;
  if constexpr (KS == 1) {
    if (q < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) yt[(4 * q + r) * NC + t * 16 + j] = y[r];
    }
    __syncthreads();
  } else {
    if (q < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((ks * T + t) * 8 + 4 * q + r) * 16 + j] = y[r];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 8 * NC; i += 64 * T * KS) {
      const int m = i / NC, c = i - m * NC;
      const int tt = c >> 4, jj = c & 15;
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < KS; ++k) sum = sum + red[((k * T + tt) * 8 + m) * 16 + jj];
      yt[i] = sum;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Dense projections (modes of ProjEpilogue).  Workgroup tg covers rows
// tg*16T .. tg*16T + 16T - 1 (tile t: rows tg*16T + 16t + j); for kHcUpMix
// (T = 4) it covers columns tg*16 .. tg*16 + 15 of the four streams (tile t:
// rows t*H + tg*16 + j).
template <int BITS, int MODE, int T, int KS, bool XREG, int SCW>
__global__ __launch_bounds__(64 * T * KS) void dense_kernel(QWeight w,
                                                            const uint16_t* __restrict__ x,
                                                            int64_t x_stride, int M,
                                                            ProjEpilogue e) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float red[KS > 1 ? KS * T * 8 * 16 : 1];
  __shared__ float yt[8 * 16 * T];
  constexpr int NC = 16 * T;
  const int tg = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15;
  const int t = wave / KS, ks = wave - t * KS;
  const int total = w.k / sk::kSuper;
  const int k0 = total * ks / KS, steps = total * (ks + 1) / KS - k0;
  const int n = w.n;
  int row;
  if constexpr (MODE == kHcUpMix)
    row = t * e.hidden + min(tg * 16 + j, e.hidden - 1);
  else
    row = min(tg * NC + t * 16 + j, n - 1);
  const int G = w.k >> 6;
  const sk::DenseRows xr{x, x_stride, M};
  constexpr int NT = 64 * T * KS;
  ProjFinish<MODE, NC, NT> fin;
  fin.begin(e, tg, M, n);
  // slices of a staged tile hold kStageSteps / KS super-steps at most
  constexpr int BMAX = XREG ? 1 : (kStageSteps / KS > 1 ? kStageSteps / KS : 1);
  const int xbytes = XREG ? 0 : total * sk::kStepBytes;
  const float* sx = reinterpret_cast<const float*>(lds + xbytes + sk::kZeroBytes);
  sk::Stream<BITS, XREG, sk::DenseRows, BMAX, SCW> st(
      w.codes + size_t(row) * (size_t(w.k) * BITS / 32), w.scales + size_t(row) * G,
      w.biases + size_t(row) * G, total, k0, steps, 0, lds, sx, xr, M);
  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (XREG) {
    st.prefetch();
    fin.prefetch(e);
    st.run(0, y);
  } else {
    sk::Stager<NT, sk::stage_per(NT, kStageSteps), sk::DenseRows> stg(xr, M, 0, total);
    stg.load();
    st.prefetch();
    fin.prefetch(e);
    stg.store(lds);
    st.run(xbytes, y);
  }
  reduce_tiles<T, KS>(y, red, yt);
  fin.finish(yt, e, tg, M, n);
}

// ---------------------------------------------------------------------------
// Expert routes.  Route r (blockIdx.y < rows*top_k) leads a chunk when the
// number of earlier routes naming its expert is a multiple of 8; the leader
// serves itself and the next up to seven routes of that expert, so every
// selected expert's weights stream once per call (one chunk per distinct
// expert when rows <= 8).  blockIdx.y == rows*top_k is the shared expert,
// serving every row.  Expert ids are clamped to the bank.
struct Routes {
  int expert;       // -1: shared expert
  int M;
  uint64_t packed;  // member m: (row << 5 | slot) at bit 8 m
};

__device__ __forceinline__ bool resolve_routes(const uint32_t* __restrict__ ids, int rows,
                                               int top_k, int experts, Routes& rt) {
  const int routes = rows * top_k;
  const int r = blockIdx.y;
  if (r == routes) {
    rt.expert = -1;
    rt.M = rows;
    rt.packed = 0;
    for (int m = 0; m < rows; ++m) rt.packed |= uint64_t((m << 5) | top_k) << (8 * m);
    return true;
  }
  const uint32_t last = uint32_t(experts - 1);
  const int lane = threadIdx.x & 63;
  // unconditional loads at clamped indices (one round trip for all three)
  const uint32_t raw0 = ids[min(lane, routes - 1)];
  const uint32_t raw1 = ids[min(64 + lane, routes - 1)];
  const uint32_t e = min(ids[r], last);
  const uint32_t id0 = lane < routes ? min(raw0, last) : 0xffffffffu;
  const uint32_t id1 = 64 + lane < routes ? min(raw1, last) : 0xffffffffu;
  uint64_t eq0 = __ballot(id0 == e);
  uint64_t eq1 = __ballot(id1 == e);
  const int before = r < 64 ? __popcll(eq0 & ((1ull << r) - 1ull))
                            : __popcll(eq0) + __popcll(eq1 & ((1ull << (r - 64)) - 1ull));
  if (before % 8 != 0) return false;
  // members: the first 8 routes u >= r naming e
  if (r < 64) {
    eq0 &= ~((1ull << r) - 1ull);
  } else {
    eq0 = 0;
    eq1 &= ~((1ull << (r - 64)) - 1ull);
  }
  rt.expert = int(e);
  rt.M = 0;
  rt.packed = 0;
  while (rt.M < 8 && (eq0 | eq1)) {
    int u;
    if (eq0) {
      u = __builtin_ctzll(eq0);
      eq0 &= eq0 - 1;
    } else {
      u = 64 + __builtin_ctzll(eq1);
      eq1 &= eq1 - 1;
    }
    const int row = u / top_k;
    rt.packed |= uint64_t((row << 5) | (u - row * top_k)) << (8 * rt.M);
    rt.M += 1;
  }
  return true;
}

__device__ __forceinline__ QWeight expert_weight(const QBank& b, int expert, const QWeight& shared) {
  if (expert < 0) return shared;
  const size_t cs = size_t(b.n) * b.k * b.bits / 32;
  const size_t ss = size_t(b.n) * (b.k / b.group_size);
  return QWeight{b.codes + cs * expert, b.scales + ss * expert, b.biases + ss * expert, b.n, b.k,
                 b.bits, b.group_size};
}

// gate/up + SwiGLU: tile 0,1 = gate rows tg*32 + 16t + j, tiles 2,3 = up rows
// of the same indices, each split along K among KS waves (wave = 4-tile
// index * KS + slice).  h[row][slot][i] = bf16(bf16(silu(bf16 g)) * bf16 u).
template <int BITS, int KS>
__global__ __launch_bounds__(256 * KS, 2) void gate_up_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ ids, int rows, int top_k,
    QBank gate, QBank up, QWeight sgate, QWeight sup, uint16_t* __restrict__ h, int hs) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float red[KS > 1 ? KS * 4 * 8 * 16 : 1];
  __shared__ float yt[8 * 64];
  Routes rt;
  if (!resolve_routes(ids, rows, top_k, gate.experts, rt)) return;
  const QWeight gw = expert_weight(gate, rt.expert, sgate);
  const QWeight uw = expert_weight(up, rt.expert, sup);
  const int inter = gw.n, hidden = gw.k;
  const int tg = blockIdx.x;
  if (tg * 32 >= inter) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15;
  const int t = wave / KS, ks = wave - t * KS;
  const bool is_gate = t < 2;
  const uint32_t* codes = is_gate ? gw.codes : uw.codes;
  const uint16_t* scales = is_gate ? gw.scales : uw.scales;
  const uint16_t* biases = is_gate ? gw.biases : uw.biases;
  const int row = min(tg * 32 + (t & 1) * 16 + j, inter - 1);
  const int G = hidden >> 6;
  const int steps = hidden / sk::kSuper;
  const int k0 = steps * ks / KS, n = steps * (ks + 1) / KS - k0;
  const sk::RouteRows xr{x, hidden, 0, rt.packed, rt.M};
  const int xbytes = steps * sk::kStepBytes;
  const float* sx = reinterpret_cast<const float*>(lds + xbytes + sk::kZeroBytes);
  sk::Stream<BITS, false, sk::RouteRows, kStageSteps / KS> st(
      codes + size_t(row) * (size_t(hidden) * BITS / 32), scales + size_t(row) * G,
      biases + size_t(row) * G, steps, k0, n, 0, lds, sx, xr, rt.M);
  sk::Stager<256 * KS, sk::stage_per(256 * KS, kStageSteps), sk::RouteRows> stg(xr, rt.M, 0,
                                                                               steps);
  stg.load();
  st.prefetch();
  stg.store(lds);
  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  st.run(xbytes, y);
  reduce_tiles<4, KS>(y, red, yt);
  if (threadIdx.x >= 256) return;
  const int m = threadIdx.x >> 5, c = threadIdx.x & 31;
  const int i = tg * 32 + c;
  if (m >= rt.M || i >= inter) return;
  const float gv = round_bf16(yt[m * 64 + c]);
  const float uv = round_bf16(yt[m * 64 + 32 + c]);
  const float silu = round_bf16(gv * sigmoid_bf16(gv));
  h[(size_t(xr.row(m)) * (top_k + 1) + xr.slot(m)) * hs + i] = f32_to_bf16(silu * uv);
}

// ---------------------------------------------------------------------------
// Persistent gate/up + SwiGLU over the distinct experts of a step.
//
// Every workgroup (4 waves) stages all rows of x once, and builds in LDS the
// list of distinct experts named by the routes (first route naming an expert
// leads; each leader carries a row mask and the slot of every member row) plus
// the shared expert.  Work items are (list entry, 32-column group); workgroup
// w takes items w, w + P, w + 2P, ... and loads the next item's weights
// before it computes the current one, so the memory system keeps streaming
// while the matrix cores and VALUs work.  Waves 2 t and 2 t + 1 compute tile t
// of the item (0, 1: gate rows 32 g + 16 t + j; 2, 3: the same up rows), one
// half of the depth each, for all eight staged rows; only member rows are
// written:
// h[row][slot][i] = bf16(bf16(silu(bf16 g)) * bf16 u), silu with the hardware
// exp2 / reciprocal.
constexpr int kPersistMaxExperts = 512;

constexpr int kPersistMaxRoutes = 128;

__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// Builds the leader list (lead_e: expert or -1 for the shared expert;
// lead_info: bit m = row m is a member, bits 8 + 5 m .. : its slot).  Returns
// the entry count.  Ends with a barrier.
// my_id: ids[threadIdx.x] for threads below rows * top_k (loaded by the caller
// at kernel start).  route_e: LDS [kPersistMaxRoutes] for the clamped ids.
__device__ __forceinline__ int build_leaders(uint32_t my_id, int rows, int top_k, int experts,
                                             int* first, unsigned long long* info, int* route_e,
                                             int* lead_e, unsigned long long* lead_info,
                                             int* count) {
  const int routes = rows * top_k;
  for (int e = threadIdx.x; e < experts; e += blockDim.x) {
    first[e] = 0x7fffffff;
    info[e] = 0ull;
  }
  __syncthreads();
  if (int(threadIdx.x) < routes) {
    const int u = threadIdx.x;
    const int e = int(min(my_id, uint32_t(experts - 1)));
    const int row = u / top_k, slot = u - row * top_k;
    route_e[u] = e;
    atomicMin(&first[e], u);
    atomicOr(&info[e], (1ull << row) | (static_cast<unsigned long long>(slot) << (8 + 5 * row)));
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int base = 0;
    for (int u0 = 0; u0 < routes; u0 += 64) {
      const int u = u0 + lane;
      const int e = u < routes ? route_e[u] : 0;
      const bool lead = u < routes && first[e] == u;
      const uint64_t bal = __ballot(lead);
      if (lead) {
        const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
        lead_e[pos] = e;
        lead_info[pos] = info[e];
      }
      base += __popcll(bal);
    }
    if (lane == 0) {
      unsigned long long all = 0;
      for (int m = 0; m < rows; ++m)
        all |= (1ull << m) | (static_cast<unsigned long long>(top_k) << (8 + 5 * m));
      lead_e[base] = -1;
      lead_info[base] = all;
      *count = base + 1;
    }
  }
  __syncthreads();
  return *count;
}

// Persistent expert gate/up.  An item is one leader expert's 16 * TPI / 2
// intermediate rows of gate and the same rows of up: TPI 16-row tiles, the
// first half gate, the second up.  KS waves share a tile, each taking 1/KS of
// the depth; a workgroup is TPI * KS waves and walks the items
// blockIdx.x, blockIdx.x + P, ... with the next item's weights in flight
// while the current one computes.
//
// PER > 0: the kernel routes its rows itself from the router logits (wave r
// routes row r with rt::route_row<PER>, PER * 64 experts); workgroup 0 writes
// the ids, scores and shared-expert factors for the kernels after it.
// PER == 0: the routes come in `ids`.
template <int BITS, int STEPS, int TPI, int KS, int PER>
__global__ __launch_bounds__(64 * TPI * KS) void gate_up_persist_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ ids, int rows, int top_k,
    QBank gate, QBank up, QWeight sgate, QWeight sup, uint16_t* __restrict__ h, int hs,
    RouteIO ro) {
  static_assert(TPI == 2 || TPI == 4, "tiles per item");
  static_assert(PER == 0 || TPI * KS >= 8, "a routing wave per row");
  constexpr int HALF = TPI / 2;   // tiles of gate (and of up) per item
  constexpr int C = 16 * HALF;    // intermediate rows (h columns) per item
  constexpr int RED = KS * TPI * 8 * 16;
  constexpr int NT = 64 * TPI * KS;
  extern __shared__ __align__(16) char lds[];
  __shared__ int first[kPersistMaxExperts];
  __shared__ unsigned long long info[kPersistMaxExperts];
  __shared__ int route_e[kPersistMaxRoutes];
  __shared__ int lead_e[kPersistMaxRoutes + 1];
  __shared__ unsigned long long lead_info[kPersistMaxRoutes + 1];
  __shared__ int count;
  // partial sums, alternating between two halves item by item: an item's
  // epilogue reads one half while the next item writes the other, so one
  // barrier per item separates writers from readers
  __shared__ float red[2 * RED];
  constexpr int steps = STEPS;  // hidden = 128 STEPS
  constexpr int hidden = STEPS * sk::kSuper;
  constexpr int G = hidden / 64;
  constexpr int xbytes = steps * sk::kStepBytes;
  const int inter = gate.n;
  const float* sx = reinterpret_cast<const float*>(lds + xbytes + sk::kZeroBytes);
  const sk::DenseRows xr{x, hidden, rows};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15;
  uint32_t my_id;
  if constexpr (PER > 0) {
    // every row is routed by a wave (its logit loads are the first ones out)
    __shared__ uint32_t routed[kPersistMaxRoutes];
    if (wave < rows) {
      const rt::RouteLane r = rt::route_row<PER>(ro.logits + size_t(wave) * ro.logit_stride, top_k);
      if (lane < top_k) {
        routed[wave * top_k + lane] = r.id;
        if (blockIdx.x == 0) {
          ro.ids[wave * top_k + lane] = r.id;
          ro.scores[wave * top_k + lane] = r.score;
        }
      }
      if (lane == 0 && blockIdx.x == 0)
        ro.factor[wave] = f32_to_bf16(
            sigmoid_bf16(bf16_to_f32(ro.shared_logit[size_t(wave) * ro.shared_stride])));
    }
    __syncthreads();
    my_id = routed[min(int(threadIdx.x), rows * top_k - 1)];
  } else {
    // route ids first (the expert list needs them), then the x staging loads
    my_id = ids[min(int(threadIdx.x), rows * top_k - 1)];
  }
  sk::Stager<NT, sk::stage_per(NT, STEPS), sk::DenseRows> stg(xr, rows, 0, steps);
  stg.load();
  const int nlead = build_leaders(my_id, rows, top_k, gate.experts, first, info, route_e, lead_e,
                                  lead_info, &count);
  const int groups = inter / C;
  const int items = nlead * groups;
  const int P = gridDim.x;
  const int t = wave / KS, ks = wave - t * KS;
  constexpr int n = steps / KS;
  const int k0 = n * ks;
  // weight rows of item `it` for this wave (tile t, depth slice ks); past the
  // last item, item `near` again: one just loaded, so its lines are still in
  // the cache and the loads stay unconditional without new HBM traffic
  auto stream_for = [&](int it, int near) {
    if (it >= items) it = near;
    const int lead = it / groups, g = it - lead * groups;
    const int e = lead_e[lead];
    const QWeight w = expert_weight(t < HALF ? gate : up, e, t < HALF ? sgate : sup);
    const int row = g * C + (t % HALF) * 16 + j;
    return sk::Stream<BITS, false, sk::DenseRows, n, 16>(
        w.codes + size_t(row) * (size_t(hidden) * BITS / 32), w.scales + size_t(row) * G,
        w.biases + size_t(row) * G, steps, k0, n, 0, lds, sx, xr, rows);
  };
  int half = 0;
  auto finish = [&](int it, float (&y)[4]) {
    sk::join_parities(y);
    float* rb = red + half * RED;
    if ((lane >> 4) < 2) {
      const int q = lane >> 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) rb[((ks * TPI + t) * 8 + 4 * q + r) * 16 + j] = y[r];
    }
    __syncthreads();
    const int lead = it / groups, g = it - lead * groups;
    const unsigned long long inf = lead_info[lead];
    if (threadIdx.x < 8 * C) {
      const int m = threadIdx.x / C, c = threadIdx.x % C;
      if ((inf >> m) & 1ull) {
        const int slot = int((inf >> (8 + 5 * m)) & 31ull);
        const int tt = c >> 4, jj = c & 15;
        float gs = 0.0f, us = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          gs = gs + rb[((k * TPI + tt) * 8 + m) * 16 + jj];
          us = us + rb[((k * TPI + HALF + tt) * 8 + m) * 16 + jj];
        }
        const float gv = round_bf16(gs);
        const float uv = round_bf16(us);
        const float silu = round_bf16(gv * sigmoid_fast(gv));
        h[(size_t(m) * (top_k + 1) + slot) * hs + g * C + c] = f32_to_bf16(silu * uv);
      }
    }
    half ^= 1;
  };
  auto step = [&](auto& st, int it) {
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    st.run(xbytes, y);
    finish(it, y);
  };
  if (int(blockIdx.x) >= items) return;  // uniform
  // the first item's weights go out before the staged x is written
  auto sa = stream_for(blockIdx.x, blockIdx.x);
  sa.prefetch();
  stg.store(lds);
  auto sb = stream_for(blockIdx.x + P, blockIdx.x);
  sb.prefetch();
  for (int it = blockIdx.x; it < items; it += 2 * P) {
    const int ib = it + P < items ? it + P : it;  // the last item loaded
    step(sa, it);
    sa = stream_for(it + 2 * P, ib);
    sa.prefetch();
    if (it + P < items) step(sb, it + P);
    sb = stream_for(it + 3 * P, it + 2 * P < items ? it + 2 * P : ib);
    sb.prefetch();
  }
}

// down + score: p[row][slot][n] = bf16(bf16(down) * score) (routed slots) or
// bf16(down) (the shared slot, top_k).  STEPS > 0: every expert (shared one
// included) is STEPS super-steps deep, all loaded in one batch; STEPS == 0:
// depths up to kDownSteps read from the bank.
template <int BITS, int STEPS>
__global__ __launch_bounds__(256, 4) void down_kernel(const uint16_t* __restrict__ h,
                                                   const uint32_t* __restrict__ ids,
                                                   const uint16_t* __restrict__ scores, int rows,
                                                   int top_k, QBank down, QWeight sdown,
                                                   uint16_t* __restrict__ p, int hs) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float yt[8 * 64];
  Routes rt;
  if (!resolve_routes(ids, rows, top_k, down.experts, rt)) return;
  const QWeight dw = expert_weight(down, rt.expert, sdown);
  const int hidden = dw.n, inter = dw.k;
  const int tg = blockIdx.x;
  if (tg * 64 >= hidden) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15;
  const int row = min(tg * 64 + wave * 16 + j, hidden - 1);
  const int G = inter >> 6;
  const int steps = STEPS > 0 ? STEPS : inter / sk::kSuper;
  const sk::RouteRows xr{h, int64_t(top_k + 1) * hs, hs, rt.packed, rt.M};
  const int xbytes = steps * sk::kStepBytes;
  const float* sx = reinterpret_cast<const float*>(lds + xbytes + sk::kZeroBytes);
  sk::Stream<BITS, false, sk::RouteRows, (STEPS > 0 ? STEPS : kDownSteps / 2), 8> st(
      dw.codes + size_t(row) * (size_t(inter) * BITS / 32), dw.scales + size_t(row) * G,
      dw.biases + size_t(row) * G, steps, 0, steps, 0, lds, sx, xr, rt.M);
  sk::Stager<256, sk::stage_per(256, (STEPS > 0 ? STEPS : kDownSteps)), sk::RouteRows> stg(
      xr, rt.M, 0, steps);
  stg.load();
  st.prefetch();
  stg.store(lds);
  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  st.run(xbytes, y);
  reduce_tiles<4, 1>(y, nullptr, yt);
  for (int t = threadIdx.x; t < 512; t += 256) {
    const int m = t >> 6, c = t & 63;
    const int r = tg * 64 + c;
    if (m >= rt.M || r >= hidden) continue;
    const int row_m = xr.row(m), slot_m = xr.slot(m);
    const bool routed = slot_m < top_k;
    const float dv = round_bf16(yt[t]);
    const float sc = routed ? bf16_to_f32(scores[size_t(row_m) * top_k + slot_m]) : 1.0f;
    p[(size_t(row_m) * (top_k + 1) + slot_m) * hidden + r] = f32_to_bf16(routed ? dv * sc : dv);
  }
}

// ---------------------------------------------------------------------------
// Expert down + score + slot sum + hyper-connection write for 512-deep experts
// and hc == 4: one workgroup per (16 output columns, token row), so the slot
// sum of a column never leaves the workgroup.  The row's slots 0..7 and
// 8..top_k (the last one the shared expert) are staged as the eight
// activation rows of two stagings; wave w streams the 16 weight rows of the
// experts of slots w, w + 4, .. (all loads issued together) over the staging
// of its slot and keeps the slot's own D row.  Every matrix-core output row
// depends only on its own activation row, so each slot value is the one
// down_kernel computes; the slot sum and the write follow
// moe_reduce_epilogue4_kernel (reference order of moe_down_tail.metal:83-99,
// then moe_epilogue.rs:17-73): the result is bit-identical to down_kernel
// followed by that kernel.  All rows of a column tile share an XCD (grid x is
// the tile), so experts chosen by several rows and the shared expert are
// fetched from HBM once per tile.  hcs: the residual streams, updated in
// place (row r, stream s at hcs + (4 r + s) hidden).
template <int BITS, int NSL>
__global__ __launch_bounds__(256, BITS * NSL <= 18 ? 4 : 2) void down_hc_kernel(
    const uint16_t* __restrict__ h, const uint32_t* __restrict__ ids,
    const uint16_t* __restrict__ scores, const uint16_t* __restrict__ factor,
    const uint16_t* __restrict__ hc_gate, int top_k, QBank down, QWeight sdown, int hs,
    uint16_t* __restrict__ hcs) {
  constexpr int STEPS = 4;
  constexpr int G = 2 * STEPS;  // 64-value groups per weight row
  constexpr int SB = sk::stage_bytes(STEPS);
  constexpr int XB = STEPS * sk::kStepBytes;
  extern __shared__ __align__(16) char lds[];
  __shared__ float pl[4 * NSL][16];
  const int tg = blockIdx.x, row = blockIdx.y;
  const int S = top_k + 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;
  const int hidden = sdown.n;
  const int col = tg * 16 + j;  // hidden % 16 == 0 (host)
  // the row's routes: one clamped slot per lane (vector loads)
  const int ls = min(lane, top_k - 1);
  const uint32_t idl = min(ids[size_t(row) * top_k + ls], uint32_t(down.experts - 1));
  const uint32_t scl = scores[size_t(row) * top_k + ls];
  // the epilogue's inputs (thread (stream es, column ec) of the first wave)
  // go out with the first loads
  const int es = (threadIdx.x >> 4) & 3, ec = threadIdx.x & 15;
  uint16_t* o = hcs + (size_t(row) * 4 + es) * hidden + tg * 16 + ec;
  const uint16_t rv = *o;
  const uint16_t fv = factor[row];
  const uint16_t gv = hc_gate[size_t(row) * 4 + es];
  const sk::DenseRows xa{h + size_t(row) * S * hs, hs, S < 8 ? S : 8};
  const sk::DenseRows xb{h + (size_t(row) * S + 8) * hs, hs, S > 8 ? S - 8 : 1};
  sk::Stager<256, sk::stage_per(256, STEPS), sk::DenseRows> sta(xa, xa.M, 0, STEPS);
  sk::Stager<256, sk::stage_per(256, STEPS), sk::DenseRows> stb(xb, xb.M, 0, STEPS);
  sta.load();
  if (S > 8) stb.load();  // uniform
  typedef sk::Stream<BITS, false, sk::DenseRows, STEPS, 8> St;
  // slot i of this wave (clamped to the last slot: a wave with fewer slots
  // re-reads the shared expert's rows and discards them)
  auto make = [&](int i) {
    const int sl = min(wave + 4 * i, S - 1);
    const int e = sl < top_k ? __shfl(int(idl), sl, 64) : -1;
    const QWeight dw = expert_weight(down, e, sdown);
    const char* base = lds + (sl >= 8 ? SB : 0);
    return St(dw.codes + size_t(col) * (size_t(STEPS) * sk::kSuper * BITS / 32),
              dw.scales + size_t(col) * G, dw.biases + size_t(col) * G, STEPS, 0, STEPS, 0,
              base, reinterpret_cast<const float*>(base + XB + sk::kZeroBytes), xa, 8);
  };
  St s0 = make(0);
  s0.prefetch();
  St s1 = make(NSL > 1 ? 1 : 0);
  if constexpr (NSL > 1) s1.prefetch();
  St s2 = make(NSL > 2 ? 2 : 0);
  if constexpr (NSL > 2) s2.prefetch();
  St s3 = make(NSL > 3 ? 3 : 0);
  if constexpr (NSL > 3) s3.prefetch();
  sta.store(lds);
  if (S > 8) stb.store(lds + SB);
  // the slot's D row m = slot % 8 sits, after the parity join, in lane
  // 16 (m / 4) + j, element m % 4; p = bf16(bf16(down) * score) for routed
  // slots, bf16(down) for the shared one
  auto finish = [&](St& st, int i) {
    const int sl = wave + 4 * i;
    if (sl >= S) return;  // uniform
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    st.run(XB, y);
    sk::join_parities(y);
    const int m = sl & 7, r = m & 3;
    const float v = r == 0 ? y[0] : r == 1 ? y[1] : r == 2 ? y[2] : y[3];
    // the score shuffle runs on every lane: its source lane may lie outside
    // the writing lanes
    const uint32_t sc = uint32_t(__shfl(int(scl), sl < top_k ? sl : 0, 64));
    if (q == (m >> 2)) {
      const float dv = round_bf16(v);
      pl[sl][j] = sl < top_k ? round_bf16(dv * bf16_to_f32(uint16_t(sc))) : dv;
    }
  };
  finish(s0, 0);
  if constexpr (NSL > 1) finish(s1, 1);
  if constexpr (NSL > 2) finish(s2, 2);
  if constexpr (NSL > 3) finish(s3, 3);
  __syncthreads();
  if (threadIdx.x >= 64) return;
  // thread (stream es, column ec): the slot sum, then the stream's write
  const int c = ec;
  const int lanes = top_k < 8 ? top_k : 8;
  float routed = 0.0f;
  for (int a = 0; a < lanes; ++a) {
    float v = pl[a][c];
    if (a + 8 < top_k) v = round_bf16(v + pl[a + 8][c]);
    routed = a == 0 ? v : round_bf16(v + routed);
  }
  routed = round_bf16(routed);
  const float combined = round_bf16(routed + round_bf16(pl[top_k][c] * bf16_to_f32(fv)));
  const float inj = round_bf16(combined * bf16_to_f32(gv));
  *o = f32_to_bf16(bf16_to_f32(rv) + inj);
}

// ---------------------------------------------------------------------------
// Greedy head: per activation row, the best (bf16(logit), lowest id) of the
// workgroup's 64 rows.  NaN never wins; a part with nothing above -inf keeps
// id 0xffffffff and -inf.
__device__ __forceinline__ void better(float v, uint32_t id, float& best, uint32_t& best_id) {
  if (v > best || (v == best && id < best_id)) {
    best = v;
    best_id = id;
  }
}

template <int BITS>
__global__ __launch_bounds__(256) void head_kernel(QWeight w, const uint16_t* __restrict__ x,
                                                   int M, float* __restrict__ maxima,
                                                   uint32_t* __restrict__ indices,
                                                   uint16_t* __restrict__ logits) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float yt[8 * 64];
  const int tg = blockIdx.x, parts = gridDim.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15;
  const int n = w.n, G = w.k >> 6;
  const int row = min(tg * 64 + wave * 16 + j, n - 1);
  const int steps = w.k / sk::kSuper;
  const sk::DenseRows xr{x, w.k, M};
  const int xbytes = steps * sk::kStepBytes;
  const float* sx = reinterpret_cast<const float*>(lds + xbytes + sk::kZeroBytes);
  sk::Stream<BITS, false, sk::DenseRows> st(w.codes + size_t(row) * (size_t(w.k) * BITS / 32),
                                            w.scales + size_t(row) * G, w.biases + size_t(row) * G,
                                            steps, 0, steps, 0, lds, sx, xr, M);
  sk::Stager<256, sk::stage_per(256, kStageSteps), sk::DenseRows> stg(xr, M, 0, steps);
  stg.load();
  st.prefetch();
  stg.store(lds);
  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  st.run(xbytes, y);
  reduce_tiles<4, 1>(y, nullptr, yt);
  for (int m = wave; m < M; m += 4) {
    const int r = tg * 64 + lane;
    float best = u2f(0xff800000u);
    uint32_t best_id = 0xffffffffu;
    if (r < n) {
      better(round_bf16(yt[m * 64 + lane]), uint32_t(r), best, best_id);
      // the bf16 logit the argmax ranks, when the caller wants the logits
      if (logits) logits[size_t(m) * n + r] = f32_to_bf16(yt[m * 64 + lane]);
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float v = __shfl_xor(best, o, 64);
      const uint32_t id = uint32_t(__shfl_xor(int(best_id), o, 64));
      better(v, id, best, best_id);
    }
    if (lane == 0) {
      maxima[size_t(m) * parts + tg] = best;
      indices[size_t(m) * parts + tg] = best_id;
    }
  }
}

// ---------------------------------------------------------------------------
// Launch geometry of a dense projection: KS = the smallest power of two that
// gives >= 3072 waves, with >= 1 super-step per slice and at most 16 waves
// per workgroup; T = 4 tiles when the split allows it (always 4 streams for
// kHcUpMix).
struct DenseCfg {
  int T, KS;
  bool xreg;
  int scw;  // scale-load width (16 when a row's scales are 16-byte aligned)
};

// Whether every slice of `total` super-steps split KS ways keeps its scale
// words within one load per lane quarter (Stream's coverage rule).
bool scale_cover(int total, int KS, int scw) {
  const int sq = scw / 4;
  for (int ks = 0; ks < KS; ++ks) {
    const int k0 = total * ks / KS, steps = total * (ks + 1) / KS - k0;
    if (k0 % sq + steps > 4 * sq) return false;
  }
  return true;
}

DenseCfg dense_cfg(const QWeight& w, const ProjEpilogue& e) {
  const int total = w.k / sk::kSuper;
  const bool mix = e.mode == kHcUpMix;
  const int tiles = mix ? 4 * ((e.hidden + 15) / 16) : (w.n + 15) / 16;
  const int max_ks = mix ? 4 : 16;
  // Measured at 8 rows on 4-bit weights: launches of 512+ column tiles run
  // fastest as four tiles x four K-splits per workgroup (GDN-in 8.6 us,
  // attention-in 8.3 us at K=2048); narrower ones as one tile split 8-16
  // ways, down to one super-step per slice staged or four from registers
  // (router 4.8 us, 4096x2048 5.3 us, 2048x4096 8.1 us).  Splits beyond
  // ~3000 waves per launch measured slower.
  const int scw = (w.k % 512 == 0) ? 16 : 8;
  const bool xreg = total > kStageSteps;
  const int min_steps = xreg ? 4 : 1;
  const int ks_cap = tiles >= 512 ? 4 : max_ks;
  int KS = 1;
  // rows with 8-byte scale loads (K % 512 != 0) are at most a few super-steps
  // deep and run unsplit
  while (scw == 16 && KS < ks_cap && tiles * KS < 3072 && total / (2 * KS) >= min_steps) KS *= 2;
  while (KS < max_ks && !scale_cover(total, KS, scw)) KS *= 2;
  const int T = (mix || KS <= 4) ? 4 : 1;
  return DenseCfg{T, KS, xreg, scw};
}

template <int BITS, int MODE, int T, int KS, bool XREG, int SCW>
void launch_dense(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
                  hipStream_t s) {
  const int groups = MODE == kHcUpMix ? (e.hidden + 15) / 16 : (w.n + 16 * T - 1) / (16 * T);
  const int total = w.k / sk::kSuper;
  hipLaunchKernelGGL((dense_kernel<BITS, MODE, T, KS, XREG, SCW>), dim3(groups),
                     dim3(64 * T * KS), XREG ? 0 : sk::stage_bytes(total), s, w, x, xs, m, e);
}

template <int BITS, int MODE>
int dense_shape(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
                hipStream_t s) {
  const DenseCfg c = dense_cfg(w, e);
  if (!scale_cover(w.k / sk::kSuper, c.KS, c.scw)) return MX_EUNSUPPORTED;
#define MX_SHAPE(T_, KS_, X_, W_)                                             \
  if (c.T == T_ && c.KS == KS_ && c.xreg == X_ && c.scw == W_) {             \
    launch_dense<BITS, MODE, T_, KS_, X_, W_>(w, x, xs, m, e, s);            \
    return MX_OK;                                                            \
  }
  MX_SHAPE(4, 1, false, 16) MX_SHAPE(4, 2, false, 16) MX_SHAPE(4, 4, false, 16)
  MX_SHAPE(4, 1, false, 8)
  MX_SHAPE(4, 2, true, 16) MX_SHAPE(4, 4, true, 16)
  if constexpr (MODE != kHcUpMix) {
    MX_SHAPE(1, 8, false, 16) MX_SHAPE(1, 16, false, 16) MX_SHAPE(1, 8, true, 16)
    MX_SHAPE(1, 16, true, 16)
  }
#undef MX_SHAPE
  return MX_EUNSUPPORTED;
}

template <int BITS>
int dense_mode(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
               hipStream_t s) {
  switch (e.mode) {
    case kPlain: return dense_shape<BITS, kPlain>(w, x, xs, m, e, s);
    case kHcDown: return dense_shape<BITS, kHcDown>(w, x, xs, m, e, s);
    case kHcUpMix: return dense_shape<BITS, kHcUpMix>(w, x, xs, m, e, s);
    case kConv:
      // conv channels come from 4-bit projections (one shape family compiled)
      if constexpr (BITS == 4) {
        if (e.taps < 2 || e.taps > kConvMaxTaps) return MX_EUNSUPPORTED;
        return dense_shape<BITS, kConv>(w, x, xs, m, e, s);
      } else {
        return MX_EUNSUPPORTED;
      }
    default: return dense_shape<BITS, kHcWrite>(w, x, xs, m, e, s);
  }
}

}  // namespace

// Scale rows must start 16-byte aligned for 16-byte scale loads
// (K % 512 == 0); rows up to 1024 deep may use 8-byte loads (K % 256 == 0).
bool skinny_supported(const QWeight& w) {
  return w.group_size == 64 && (w.k % 512 == 0 || (w.k % 256 == 0 && w.k <= 1024)) &&
         w.k / sk::kSuper <= kDenseSteps &&
         (w.bits == 4 || w.bits == 5 || w.bits == 6 || w.bits == 8);
}

int skinny_dense(const QWeight& w, const uint16_t* x, int64_t x_stride, int m,
                 const ProjEpilogue& e, hipStream_t s) {
  if (!skinny_supported(w) || m < 1 || m > 8) return MX_EUNSUPPORTED;
  if (e.mode == kHcUpMix && e.hidden * 4 != w.n) return MX_EUNSUPPORTED;
  int rc;
  switch (w.bits) {
    case 4: rc = dense_mode<4>(w, x, x_stride, m, e, s); break;
    case 5: rc = dense_mode<5>(w, x, x_stride, m, e, s); break;
    case 6: rc = dense_mode<6>(w, x, x_stride, m, e, s); break;
    default: rc = dense_mode<8>(w, x, x_stride, m, e, s); break;
  }
  if (rc != MX_OK) return rc;
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

namespace {

bool persist_ok(const QBank& gate, const QBank& up, const QWeight& sgate, int rows, int top_k) {
  return gate.experts <= kPersistMaxExperts && rows * top_k <= kPersistMaxRoutes &&
         sgate.n == gate.n && up.n == gate.n && gate.n % (8 * kPersistTiles) == 0 &&
         gate.k / sk::kSuper == kStageSteps;
}

// One workgroup per resident slot: every workgroup is on the chip from the start.
template <int BITS, int PER>
int launch_persist(const uint16_t* x, const uint32_t* ids, int rows, int top_k, const QBank& gate,
                   const QBank& up, const QWeight& sgate, const QWeight& sup, uint16_t* h, int hs,
                   const RouteIO& ro, hipStream_t s) {
  constexpr int NT = 64 * kPersistTiles * kPersistSplit;
  const auto fn = gate_up_persist_kernel<BITS, kStageSteps, kPersistTiles, kPersistSplit, PER>;
  const int lb = sk::stage_bytes(kStageSteps);
  static int grid_n = 0;
  if (grid_n == 0) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn),
                                                     NT, lb) != hipSuccess ||
        cus <= 0 || per_cu <= 0)
      return MX_EHIP;
    grid_n = cus * per_cu;
  }
  hipLaunchKernelGGL(fn, dim3(grid_n), dim3(NT), lb, s, x, ids, rows, top_k, gate, up, sgate, sup,
                     h, hs, ro);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

template <int PER>
int dispatch_persist(const uint16_t* x, const uint32_t* ids, int rows, int top_k,
                     const QBank& gate, const QBank& up, const QWeight& sgate, const QWeight& sup,
                     uint16_t* h, int hs, const RouteIO& ro, hipStream_t s) {
  switch (gate.bits) {
    case 4: return launch_persist<4, PER>(x, ids, rows, top_k, gate, up, sgate, sup, h, hs, ro, s);
    case 5: return launch_persist<5, PER>(x, ids, rows, top_k, gate, up, sgate, sup, h, hs, ro, s);
    case 6: return launch_persist<6, PER>(x, ids, rows, top_k, gate, up, sgate, sup, h, hs, ro, s);
    default: return launch_persist<8, PER>(x, ids, rows, top_k, gate, up, sgate, sup, h, hs, ro, s);
  }
}

int gate_up_check(int rows, int top_k, const QBank& gate, const QBank& up, const QWeight& sgate,
                  const QWeight& sup) {
  const int steps = gate.k / sk::kSuper;
  if (rows < 1 || rows > 8 || top_k < 1 || top_k > 16 || gate.group_size != 64 ||
      gate.k % 512 != 0 || steps > kStageSteps || up.bits != gate.bits ||
      sgate.bits != gate.bits || sup.bits != gate.bits || sgate.k != gate.k)
    return MX_EUNSUPPORTED;
  return MX_OK;
}

}  // namespace

int skinny_gate_up(const uint16_t* x, const uint32_t* ids, int rows, int top_k,
                   const QBank& gate, const QBank& up, const QWeight& sgate, const QWeight& sup,
                   uint16_t* h, hipStream_t s) {
  const int hs = gate.n > sgate.n ? gate.n : sgate.n;
  if (gate_up_check(rows, top_k, gate, up, sgate, sup) != MX_OK) return MX_EUNSUPPORTED;
  if (persist_ok(gate, up, sgate, rows, top_k))
    return dispatch_persist<0>(x, ids, rows, top_k, gate, up, sgate, sup, h, hs, RouteIO{}, s);
  const int lb = sk::stage_bytes(gate.k / sk::kSuper);
  const dim3 grid((hs + 31) / 32, rows * top_k + 1);
#define MX_GU(B) \
  case B: hipLaunchKernelGGL((gate_up_kernel<B, kGateUpSplit>), grid, dim3(256 * kGateUpSplit), lb, s, x, ids, rows, top_k, gate, up, sgate, sup, h, hs); break;
  switch (gate.bits) {
    MX_GU(4) MX_GU(5) MX_GU(6) MX_GU(8)
    default: return MX_EUNSUPPORTED;
  }
#undef MX_GU
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int skinny_route_gate_up(const RouteIO& ro, int experts, const uint16_t* x, int rows, int top_k,
                         const QBank& gate, const QBank& up, const QWeight& sgate,
                         const QWeight& sup, uint16_t* h, hipStream_t s) {
  const int hs = gate.n > sgate.n ? gate.n : sgate.n;
  if (gate_up_check(rows, top_k, gate, up, sgate, sup) != MX_OK) return MX_EUNSUPPORTED;
  if (experts == 8 * 64 && experts <= gate.experts && persist_ok(gate, up, sgate, rows, top_k))
    return dispatch_persist<8>(x, ro.ids, rows, top_k, gate, up, sgate, sup, h, hs, ro, s);
  const int rc = moe_route(ro.logits, ro.logit_stride, ro.shared_logit, ro.shared_stride, rows,
                           experts, top_k, ro.ids, ro.scores, ro.factor, s);
  if (rc != MX_OK) return rc;
  return skinny_gate_up(x, ro.ids, rows, top_k, gate, up, sgate, sup, h, s);
}

int skinny_down(const uint16_t* h, const uint32_t* ids, const uint16_t* scores, int rows,
                int top_k, int inter, int shared_inter, const QBank& down, const QWeight& sdown,
                uint16_t* p, hipStream_t s) {
  const int hs = inter > shared_inter ? inter : shared_inter;
  const int kmax = down.k > sdown.k ? down.k : sdown.k;
  if (rows < 1 || rows > 8 || top_k < 1 || top_k > 16 || down.group_size != 64 ||
      down.k % 256 != 0 || sdown.k % 256 != 0 || kmax / sk::kSuper > kDownSteps ||
      sdown.bits != down.bits || sdown.n != down.n)
    return MX_EUNSUPPORTED;
  const dim3 grid((down.n + 63) / 64, rows * top_k + 1);
  const int lb = sk::stage_bytes(kmax / sk::kSuper);
  // 512-deep experts (the common MoE shape) run with their depth fixed at
  // compile time: one batch of loads and, at 4-8 bits, 60-66 VGPRs (twice
  // the resident waves of the general form)
  const bool d4 = down.k == 4 * sk::kSuper && sdown.k == 4 * sk::kSuper;
#define MX_DN(B)                                                                            \
  case B:                                                                                   \
    if (d4)                                                                                 \
      hipLaunchKernelGGL((down_kernel<B, 4>), grid, dim3(256), lb, s, h, ids, scores, rows, \
                         top_k, down, sdown, p, hs);                                        \
    else                                                                                    \
      hipLaunchKernelGGL((down_kernel<B, 0>), grid, dim3(256), lb, s, h, ids, scores, rows, \
                         top_k, down, sdown, p, hs);                                        \
    break;
  switch (down.bits) {
    MX_DN(4) MX_DN(5) MX_DN(6) MX_DN(8)
    default: return MX_EUNSUPPORTED;
  }
#undef MX_DN
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

bool skinny_down_hc_supported(int rows, int top_k, int hc, const QBank& down,
                              const QWeight& sdown) {
  return rows >= 1 && rows <= 8 && top_k >= 1 && top_k + 1 <= 16 && hc == 4 &&
         down.group_size == 64 && sdown.group_size == 64 && down.k == 4 * sk::kSuper &&
         sdown.k == 4 * sk::kSuper && sdown.bits == down.bits && sdown.n == down.n &&
         down.n % 16 == 0 && down.experts >= 1 &&
         (down.bits == 4 || down.bits == 5 || down.bits == 6 || down.bits == 8);
}

int skinny_down_hc(const uint16_t* h, const uint32_t* ids, const uint16_t* scores,
                   const uint16_t* factor, const uint16_t* hc_gate, int rows, int top_k, int hc,
                   int inter, int shared_inter, const QBank& down, const QWeight& sdown,
                   uint16_t* hcs, hipStream_t s) {
  if (!skinny_down_hc_supported(rows, top_k, hc, down, sdown)) return MX_EUNSUPPORTED;
  const int hs = inter > shared_inter ? inter : shared_inter;
  const int nsl = (top_k + 1 + 3) / 4;
  const dim3 grid(down.n / 16, rows);
  const int lb = 2 * sk::stage_bytes(4);
  switch (down.bits * 8 + nsl) {
#define MX_DH(B, N)                                                                          \
  case B * 8 + N:                                                                            \
    hipLaunchKernelGGL((down_hc_kernel<B, N>), grid, dim3(256), lb, s, h, ids, scores, factor, \
                       hc_gate, top_k, down, sdown, hs, hcs);                                 \
    break;
    MX_DH(4, 1) MX_DH(4, 2) MX_DH(4, 3) MX_DH(4, 4) MX_DH(5, 1) MX_DH(5, 2) MX_DH(5, 3)
    MX_DH(5, 4) MX_DH(6, 1) MX_DH(6, 2) MX_DH(6, 3) MX_DH(6, 4) MX_DH(8, 1) MX_DH(8, 2)
    MX_DH(8, 3) MX_DH(8, 4)
#undef MX_DH
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int skinny_head_parts(int n) { return (n + 63) / 64; }

int skinny_head(const QWeight& w, const uint16_t* x, int m, float* maxima, uint32_t* indices,
                int* parts_out, hipStream_t s, uint16_t* logits) {
  if (!skinny_supported(w) || m < 1 || m > 8 || w.k % 512 != 0 || w.k / sk::kSuper > kStageSteps)
    return MX_EUNSUPPORTED;
  const int parts = skinny_head_parts(w.n);
  *parts_out = parts;
  const int lb = sk::stage_bytes(w.k / sk::kSuper);
  switch (w.bits) {
    case 4: hipLaunchKernelGGL(head_kernel<4>, dim3(parts), dim3(256), lb, s, w, x, m, maxima, indices, logits); break;
    case 5: hipLaunchKernelGGL(head_kernel<5>, dim3(parts), dim3(256), lb, s, w, x, m, maxima, indices, logits); break;
    case 6: hipLaunchKernelGGL(head_kernel<6>, dim3(parts), dim3(256), lb, s, w, x, m, maxima, indices, logits); break;
    default: hipLaunchKernelGGL(head_kernel<8>, dim3(parts), dim3(256), lb, s, w, x, m, maxima, indices, logits); break;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
