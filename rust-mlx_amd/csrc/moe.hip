// Sparse-MoE decode kernels for gfx950: routing tail, gathered expert
// gate/up (+SwiGLU), gathered down (+score), and the slot reduction fused with
// the hyper-connection epilogue.
//
// Reference: MoE::parts (src/hybrid.rs:192-287), moe_route::tail
// (src/moe_route.rs:25-70, kernels/moe_route_tail.{h,metal}), moe_kernel::gate_up
// (src/moe_kernel.rs:10-118, kernels/moe_gate_up{4,5}.metal), moe_down::reduce
// (src/moe_down.rs:34-137, kernels/moe_down_tail.{h,metal}) and
// moe_epilogue::apply (src/moe_epilogue.rs:17-73, kernels/moe_hc_epilogue.metal).
//
// Expert deduplication: every (row, slot) route of one step that names the same
// expert is served by the workgroup of the expert's first route, so each
// selected expert's weights stream from HBM once per step however many rows
// chose it (the reference gathers per route, moe_kernel.rs:100-113).
#include "common.hpp"
#include "kernels.hpp"
#include "qmv_core.hpp"
#include "route_core.hpp"
#include "xq_core.hpp"

namespace mx {

namespace {

constexpr int kWaves = 4;

// ---------------------------------------------------------------------------
// Routing tail: softmax (fp32, MLX precise) -> bf16 gates -> top-k under the
// (bf16 value, index) key -> bf16 renormalisation -> bf16 sigmoid of the
// shared-expert gate.  One wave per row (rt::route_row).
template <int PER>
__global__ __launch_bounds__(64) void route_kernel(const uint16_t* __restrict__ logits,
                                                   int64_t logit_stride,
                                                   const uint16_t* __restrict__ shared_logit,
                                                   int64_t shared_stride, int experts, int top_k,
                                                   uint32_t* __restrict__ ids,
                                                   uint16_t* __restrict__ scores,
                                                   uint16_t* __restrict__ factor) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const rt::RouteLane r = rt::route_row<PER>(logits + size_t(row) * logit_stride, top_k);
  if (lane < top_k) {
    ids[size_t(row) * top_k + lane] = r.id;
    scores[size_t(row) * top_k + lane] = r.score;
  }
  if (lane == 0)
    factor[row] = f32_to_bf16(sigmoid_bf16(bf16_to_f32(shared_logit[size_t(row) * shared_stride])));
}

// ---------------------------------------------------------------------------
// Expert work plan: one entry per distinct routed expert (in order of first
// appearance among the rows' slots) plus one for the shared expert, listing
// the (row, slot) routes it serves.  One workgroup; routes <= 8 * 16 + 1.
// The plan from the route ids in sids (LDS); every thread of the workgroup
// calls it (NT threads, at most 8 waves; routes <= 8 * 16 + 1).
template <int NT>
__device__ __forceinline__ void plan_body(const uint32_t* sids, int rows, int top_k,
                                          MoePlan* __restrict__ plan) {
  __shared__ int entry_of[kMaxRoutes];  // entry index, by its first route
  __shared__ int wave_count[8], wave_items[8];
  // per expert: the rows that route to it (a bit per row) and its first
  // route; filled with LDS atomics, which need no order, so every route
  // learns its expert's routes in one pass instead of a scan of all routes
  constexpr int kTable = 1024;  // experts (at most 1024)
  __shared__ uint32_t row_mask[kTable];
  __shared__ int first_route[kTable];
  constexpr int NW = NT / 64;
  const int t = threadIdx.x;
  const int routes = rows * top_k;
  for (int i = t; i < kTable; i += NT) {
    row_mask[i] = 0u;
    first_route[i] = 1 << 30;
  }
  __syncthreads();
  const bool routed = t < routes;
  const uint32_t e = routed ? sids[t] & uint32_t(kTable - 1) : 0u;
  const int row = routed ? t / top_k : 0;
  if (routed) {
    atomicOr(&row_mask[e], 1u << row);
    atomicMin(&first_route[e], t);
  }
  __syncthreads();
  // this route's place among its expert's routes (route order: each row
  // routes to an expert at most once, so by row), how many there are, which
  // four-row blocks of rows they come from
  int first_u = t, pos = 0, cnt = 0, blkmask = 0;
  if (routed) {
    const uint32_t mask = row_mask[e];
    first_u = first_route[e];
    pos = __popc(mask & ((1u << row) - 1u));
    cnt = __popc(mask);
    blkmask = ((mask & 0x0fu) ? 1 : 0) | ((mask & 0xf0u) ? 2 : 0);
  } else if (t == routes) {  // the shared expert: every row, slot top_k
    cnt = rows;
    blkmask = rows > 4 ? 3 : 1;
  }
  const bool first = routed ? first_u == t : t == routes;
  const uint64_t mask = __ballot(first);
  const int lane = t & 63, wave = t >> 6;
  if (lane == 0) wave_count[wave] = __popcll(mask);
  // items, (entry, block with a member) pairs in entry order
  const int nb = first ? __popc(blkmask) : 0;
  const uint64_t one = __ballot(nb >= 1), two = __ballot(nb == 2);
  const uint64_t below = (1ull << lane) - 1ull;
  int pos_item = __popcll(one & below) + __popcll(two & below);
  if (lane == 0) wave_items[wave] = __popcll(one) + __popcll(two);
  __syncthreads();
  int idx = __popcll(mask & below), count = 0, nitems = 0;
  for (int w = 0; w < NW; ++w) {
    if (w < wave) {
      idx += wave_count[w];
      pos_item += wave_items[w];
    }
    count += wave_count[w];
    nitems += wave_items[w];
  }
  if (t == 0) {
    plan->count = count;
    plan->nitems = nitems;
  }
  if (first) {
    entry_of[t] = idx;
    plan->expert[idx] = routed ? int(e) : -1;
    plan->m[idx] = cnt;
    for (int b = 0; b < 2; ++b)
      if ((blkmask >> b) & 1) plan->item[pos_item++] = uint16_t(2 * idx + b);
  }
  if (t == routes)
    for (int r = 0; r < rows; ++r) {
      plan->row[idx][r] = uint8_t(r);
      plan->slot[idx][r] = uint8_t(top_k);
    }
  __syncthreads();
  if (routed) {
    const int en = entry_of[first_u];
    plan->row[en][pos] = uint8_t(t / top_k);
    plan->slot[en][pos] = uint8_t(t % top_k);
  }
}

__global__ __launch_bounds__(256) void plan_kernel(const uint32_t* __restrict__ ids, int rows,
                                                   int top_k, MoePlan* __restrict__ plan) {
  __shared__ uint32_t sids[kMaxRoutes];
  const int t = threadIdx.x;
  if (t < rows * top_k) sids[t] = ids[t];
  __syncthreads();
  plan_body<256>(sids, rows, top_k, plan);
}

// Routing tail (route_kernel's arithmetic, wave r routing row r) and the plan
// of its routes in one workgroup.
template <int PER>
__global__ __launch_bounds__(512) void route_plan_kernel(
    const uint16_t* __restrict__ logits, int64_t logit_stride,
    const uint16_t* __restrict__ shared_logit, int64_t shared_stride, int rows, int top_k,
    uint32_t* __restrict__ ids, uint16_t* __restrict__ scores, uint16_t* __restrict__ factor,
    MoePlan* __restrict__ plan) {
  __shared__ uint32_t sids[kMaxRoutes];
  const int lane = threadIdx.x & 63, row = threadIdx.x >> 6;
  if (row < rows) {
    // the shared-expert logit is requested with the row's logits, so its
    // latency overlaps theirs instead of following the top-k
    const uint16_t sh = shared_logit[size_t(row) * shared_stride];  // every lane: no branch
    const rt::RouteLane r = rt::route_row<PER>(logits + size_t(row) * logit_stride, top_k);
    if (lane < top_k) {
      ids[size_t(row) * top_k + lane] = r.id;
      scores[size_t(row) * top_k + lane] = r.score;
      sids[row * top_k + lane] = r.id;
    }
    if (lane == 0) factor[row] = f32_to_bf16(sigmoid_bf16(bf16_to_f32(sh)));
  }
  __syncthreads();
  plan_body<512>(sids, rows, top_k, plan);
}

// ---------------------------------------------------------------------------
// Expert work list of a prefill chunk (up to kPrefillChunk rows): the routes
// grouped by expert, experts in index order and then the shared expert, each
// expert's routes in row order (a row names an expert at most once), cut into
// items of at most 16 routes.  One workgroup of 1024 threads; thread e < 1024
// owns expert e (the shared expert is index `experts`).
constexpr int kChunkPlanThreads = 1024;

// Exclusive prefix sum over the workgroup's threads in thread order, and the
// total (every thread calls it).
__device__ __forceinline__ int block_exclusive_sum(int v, int* total) {
  __shared__ int wave_sum[kChunkPlanThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  if (lane == 63) wave_sum[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < kChunkPlanThreads / 64; ++w) {
    if (w < wave) before += wave_sum[w];
    all += wave_sum[w];
  }
  __syncthreads();  // wave_sum may be reused by the next call
  *total = all;
  return before + incl - v;
}

__global__ __launch_bounds__(kChunkPlanThreads) void chunk_plan_kernel(
    const uint32_t* __restrict__ ids, int rows, int experts, int top_k,
    ChunkPlan* __restrict__ plan) {
  // rows (bits 0..127) that route to each expert
  __shared__ uint32_t mask[kChunkPlanThreads][kPrefillChunk / 32];
  __shared__ int first[kChunkPlanThreads];  // each expert's first member
  const int t = threadIdx.x;
  constexpr int W = kPrefillChunk / 32;
#pragma unroll
  for (int w = 0; w < W; ++w) mask[t][w] = 0u;
  __syncthreads();
  const int routes = rows * top_k;
  for (int r = t; r < routes; r += kChunkPlanThreads) {
    const uint32_t e = ids[r];
    const int row = r / top_k;
    if (e < uint32_t(experts)) atomicOr(&mask[e][row >> 5], 1u << (row & 31));
  }
  __syncthreads();
  int cnt = 0;
  if (t < experts) {
#pragma unroll
    for (int w = 0; w < W; ++w) cnt += __popc(mask[t][w]);
  } else if (t == experts) {
    cnt = rows;
  }
  const int items = (cnt + 15) / 16;
  int members = 0, nitems = 0;
  const int m_off = block_exclusive_sum(cnt, &members);
  const int i_off = block_exclusive_sum(items, &nitems);
  first[t] = m_off;
  if (t == 0) plan->nitems = nitems;
  for (int i = 0; i < items; ++i) {
    plan->expert[i_off + i] = t == experts ? -1 : t;
    plan->start[i_off + i] = m_off + 16 * i;
    plan->m[i_off + i] = cnt - 16 * i < 16 ? cnt - 16 * i : 16;
  }
  __syncthreads();
  for (int r = t; r < routes; r += kChunkPlanThreads) {
    const uint32_t e = ids[r];
    if (e >= uint32_t(experts)) continue;
    const int row = r / top_k;
    int rank = __popc(mask[e][row >> 5] & ((1u << (row & 31)) - 1u));
    for (int w = 0; w < (row >> 5); ++w) rank += __popc(mask[e][w]);
    const int at = first[e] + rank;
    plan->row[at] = uint16_t(row);
    plan->slot[at] = uint8_t(r - row * top_k);
  }
  for (int row = t; row < rows; row += kChunkPlanThreads) {
    plan->row[first[experts] + row] = uint16_t(row);
    plan->slot[first[experts] + row] = uint8_t(top_k);
  }
}

struct Bank {
  const uint32_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  size_t code_stride, scale_stride;  // per expert
};

__device__ __forceinline__ Bank bank_for(const QBank& b, int expert, const QWeight& shared) {
  if (expert < 0) return Bank{shared.codes, shared.scales, shared.biases, 0, 0};
  const size_t cs = size_t(b.n) * b.k * b.bits / 32;
  const size_t ss = size_t(b.n) * (b.k / b.group_size);
  return Bank{b.codes + cs * expert, b.scales + ss * expert, b.biases + ss * expert, cs, ss};
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU.  h[row][slot][i] = bf16(bf16(g * sigmoid(g)) * u).
template <int BITS, int M>
__device__ void gate_up_body(const uint16_t* __restrict__ x, const Bank& gb, const Bank& ub,
                             int inter, int hidden, int gs, const int* row_of, const int* slot_of,
                             int top_k, uint16_t* __restrict__ h, int hs, int row0, int li, int L) {
  int rows[kQRows];
#pragma unroll
  for (int r = 0; r < kQRows; ++r) rows[r] = min(row0 + r, inter - 1);
  const uint16_t* xrow[M];
#pragma unroll
  for (int m = 0; m < M; ++m) xrow[m] = x + size_t(row_of[m]) * hidden;
  float g[M][kQRows], u[M][kQRows];
  qmv_core<BITS, M>(gb.codes, gb.scales, gb.biases, hidden, gs, xrow, rows, li, L, g);
  qmv_core<BITS, M>(ub.codes, ub.scales, ub.biases, hidden, gs, xrow, rows, li, L, u);
  if (li == 0) {
#pragma unroll
    for (int r = 0; r < kQRows; ++r) {
      if (row0 + r >= inter) continue;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float gv = round_bf16(g[m][r]);
        const float uv = round_bf16(u[m][r]);
        const float silu = round_bf16(gv * sigmoid_bf16(gv));
        h[(size_t(row_of[m]) * (top_k + 1) + slot_of[m]) * hs + row0 + r] =
            f32_to_bf16(silu * uv);
      }
    }
  }
}

template <int BITS>
__global__ __launch_bounds__(256) void gate_up_kernel(const uint16_t* __restrict__ x,
                                                      const MoePlan* __restrict__ plan,
                                                      int top_k, QBank gate, QBank up,
                                                      QWeight sgate, QWeight sup,
                                                      uint16_t* __restrict__ h, int hs) {
  const int entry = blockIdx.y;
  if (entry >= plan->count) return;
  const int m = plan->m[entry];
  const int expert = plan->expert[entry];
  const Bank gb = bank_for(gate, expert, sgate);
  const Bank ub = bank_for(up, expert, sup);
  const int inter = expert < 0 ? sgate.n : gate.n;
  const int hidden = gate.k;
  const int L = qmv_lanes_per_row(hidden);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & (L - 1), lg = lane / L;
  const int row0 = ((blockIdx.x * kWaves + wave) * (64 / L) + lg) * kQRows;
  if (row0 >= inter) return;
  int ro[8], so[8];
  for (int i = 0; i < 8; ++i) {
    ro[i] = plan->row[entry][i];
    so[i] = plan->slot[entry][i];
  }
  switch (m) {
#define MX_CASE(MM) \
  case MM: gate_up_body<BITS, MM>(x, gb, ub, inter, hidden, gate.group_size, ro, so, top_k, h, hs, row0, li, L); break;
    MX_CASE(1) MX_CASE(2) MX_CASE(3) MX_CASE(4) MX_CASE(5) MX_CASE(6) MX_CASE(7) MX_CASE(8)
#undef MX_CASE
  }
}

// ---------------------------------------------------------------------------
// down + score.  p[row][slot][n] = bf16(bf16(down) * score) for routed slots;
// the shared slot (top_k) keeps bf16(down).
template <int BITS, int M>
__device__ void down_body(const uint16_t* __restrict__ h, const Bank& db, int hidden, int inter,
                          int gs, const int* row_of, const int* slot_of, int top_k,
                          const uint16_t* __restrict__ scores, uint16_t* __restrict__ p, int hs,
                          int row0, int li, int L) {
  int rows[kQRows];
#pragma unroll
  for (int r = 0; r < kQRows; ++r) rows[r] = min(row0 + r, hidden - 1);
  const uint16_t* xrow[M];
#pragma unroll
  for (int m = 0; m < M; ++m)
    xrow[m] = h + (size_t(row_of[m]) * (top_k + 1) + slot_of[m]) * hs;
  float d[M][kQRows];
  qmv_core<BITS, M>(db.codes, db.scales, db.biases, inter, gs, xrow, rows, li, L, d);
  if (li == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const bool routed = slot_of[m] < top_k;
      const float sc =
          routed ? bf16_to_f32(scores[size_t(row_of[m]) * top_k + slot_of[m]]) : 1.0f;
#pragma unroll
      for (int r = 0; r < kQRows; ++r) {
        if (row0 + r >= hidden) continue;
        const float dv = round_bf16(d[m][r]);
        p[(size_t(row_of[m]) * (top_k + 1) + slot_of[m]) * hidden + row0 + r] =
            f32_to_bf16(routed ? dv * sc : dv);
      }
    }
  }
}

template <int BITS>
__global__ __launch_bounds__(256) void down_kernel(const uint16_t* __restrict__ h,
                                                   const MoePlan* __restrict__ plan,
                                                   const uint16_t* __restrict__ scores,
                                                   int top_k, QBank down, QWeight sdown,
                                                   uint16_t* __restrict__ p, int hs) {
  const int entry = blockIdx.y;
  if (entry >= plan->count) return;
  const int m = plan->m[entry];
  const int expert = plan->expert[entry];
  const Bank db = bank_for(down, expert, sdown);
  const int hidden = down.n;
  const int inter = expert < 0 ? sdown.k : down.k;
  const int L = qmv_lanes_per_row(inter);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & (L - 1), lg = lane / L;
  const int row0 = ((blockIdx.x * kWaves + wave) * (64 / L) + lg) * kQRows;
  if (row0 >= hidden) return;
  int ro[8], so[8];
  for (int i = 0; i < 8; ++i) {
    ro[i] = plan->row[entry][i];
    so[i] = plan->slot[entry][i];
  }
  switch (m) {
#define MX_CASE(MM) \
  case MM: down_body<BITS, MM>(h, db, hidden, inter, down.group_size, ro, so, top_k, scores, p, hs, row0, li, L); break;
    MX_CASE(1) MX_CASE(2) MX_CASE(3) MX_CASE(4) MX_CASE(5) MX_CASE(6) MX_CASE(7) MX_CASE(8)
#undef MX_CASE
  }
}

// ---------------------------------------------------------------------------
// Slot reduction.  routed = bf16 sum of p[row][0..k-1][c] in the reference's
// order (kernels/moe_down_tail.h:20, moe_down_tail.metal:83-99): slot i
// accumulates into lane i % 8 with one bf16 add per later slot, then lanes
// 1..7 are added to lane 0's value one by one.  For k = 10 this is the order
// {0,8},{1,9},2,3,...,7 of the reference's SLOT_ORDER.
__device__ __forceinline__ float slot_sum(const uint16_t* __restrict__ pr, int top_k,
                                          size_t stride) {
  float acc[8] = {0.0f};
  const int lanes = top_k < 8 ? top_k : 8;
  for (int a = 0; a < lanes; ++a) {
    float v = bf16_to_f32(pr[size_t(a) * stride]);
    for (int s = a + 8; s < top_k; s += 8) v = round_bf16(v + bf16_to_f32(pr[size_t(s) * stride]));
    acc[a] = v;
  }
  float routed = acc[0];
  for (int a = 1; a < lanes; ++a) routed = round_bf16(acc[a] + routed);
  return routed;
}

// Hyper-connection write of the MoE output (kernels/moe_hc_epilogue.metal:8-11):
//   weighted = bf16(shared * factor); combined = bf16(routed + weighted)
//   out[s] = bf16(residual[s] + bf16(combined * gate[s]))
__device__ __forceinline__ void hc_write(float routed, float shared, float factor,
                                         const uint16_t* __restrict__ residual,
                                         const uint16_t* __restrict__ gate, int hc, int hidden,
                                         uint16_t* __restrict__ out) {
  const float weighted = round_bf16(shared * factor);
  const float combined = round_bf16(routed + weighted);
  for (int s = 0; s < hc; ++s) {
    const float inj = round_bf16(combined * bf16_to_f32(gate[s]));
    out[size_t(s) * hidden] = f32_to_bf16(bf16_to_f32(residual[size_t(s) * hidden]) + inj);
  }
}

__global__ __launch_bounds__(256) void moe_reduce_kernel(const uint16_t* __restrict__ p,
                                                         int top_k, int hidden,
                                                         uint16_t* __restrict__ routed) {
  const int row = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= hidden) return;
  const uint16_t* pr = p + size_t(row) * (top_k + 1) * hidden + c;
  routed[size_t(row) * hidden + c] = f32_to_bf16(slot_sum(pr, top_k, hidden));
}

__global__ __launch_bounds__(256) void moe_epilogue_kernel(
    const uint16_t* __restrict__ routed, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ factor, const uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ gate, int hc, int hidden, uint16_t* __restrict__ out) {
  const int row = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= hidden) return;
  const size_t o = size_t(row) * hc * hidden + c;
  hc_write(bf16_to_f32(routed[size_t(row) * hidden + c]),
           bf16_to_f32(shared[size_t(row) * hidden + c]), bf16_to_f32(factor[row]),
           residual + o, gate + size_t(row) * hc, hc, hidden, out + o);
}

__global__ __launch_bounds__(256) void moe_reduce_epilogue_kernel(
    const uint16_t* __restrict__ p, const uint16_t* __restrict__ factor,
    const uint16_t* __restrict__ residual, const uint16_t* __restrict__ gate, int top_k, int hc,
    int hidden, uint16_t* __restrict__ out) {
  const int row = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= hidden) return;
  const uint16_t* pr = p + size_t(row) * (top_k + 1) * hidden + c;
  // the reduced value is rounded to bf16 exactly as the separate kernels store it
  const float routed = round_bf16(slot_sum(pr, top_k, hidden));
  const size_t o = size_t(row) * hc * hidden + c;
  hc_write(routed, bf16_to_f32(pr[size_t(top_k) * hidden]), bf16_to_f32(factor[row]),
           residual + o, gate + size_t(row) * hc, hc, hidden, out + o);
}

// The same arithmetic for 4 consecutive columns per thread, with every load
// issued before the first add (slot values for k <= 15 at clamped slot
// indices, the shared slot, residual and gates); hc == 4.
constexpr int kRedMaxK = 16;
__global__ __launch_bounds__(256) void moe_reduce_epilogue4_kernel(
    const uint16_t* __restrict__ p, const uint16_t* __restrict__ factor,
    const uint16_t* __restrict__ residual, const uint16_t* __restrict__ gate, int top_k,
    int hidden, uint16_t* __restrict__ out) {
  constexpr int HC = 4;
  const int row = blockIdx.y;
  const int c = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (c >= hidden) return;
  const uint16_t* pr = p + size_t(row) * (top_k + 1) * hidden + c;
  uint2 pv[kRedMaxK];
#pragma unroll
  for (int sl = 0; sl < kRedMaxK; ++sl)
    pv[sl] = *reinterpret_cast<const uint2*>(pr + size_t(sl < top_k ? sl : top_k) * hidden);
  const uint2 sh = *reinterpret_cast<const uint2*>(pr + size_t(top_k) * hidden);
  const size_t o = size_t(row) * HC * hidden + c;
  uint2 rv[HC];
  float gv[HC];
#pragma unroll
  for (int s2 = 0; s2 < HC; ++s2) {
    rv[s2] = *reinterpret_cast<const uint2*>(residual + o + size_t(s2) * hidden);
    gv[s2] = bf16_to_f32(gate[size_t(row) * HC + s2]);
  }
  const float f = bf16_to_f32(factor[row]);
  const int lanes = top_k < 8 ? top_k : 8;
  uint16_t res[HC][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    auto col = [&](const uint2& v) {
      return bf16_to_f32(uint16_t(i < 2 ? (v.x >> (16 * i)) : (v.y >> (16 * (i - 2)))));
    };
    // slot_sum with compile-time register indices (predicated by top_k)
    float acc[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      float v = col(pv[a]);
      if (a + 8 < top_k) v = round_bf16(v + col(pv[a + 8]));
      acc[a] = v;
    }
    float routed = acc[0];
#pragma unroll
    for (int a = 1; a < 8; ++a)
      if (a < lanes) routed = round_bf16(acc[a] + routed);
    routed = round_bf16(routed);
    const float weighted = round_bf16(col(sh) * f);
    const float combined = round_bf16(routed + weighted);
#pragma unroll
    for (int s2 = 0; s2 < HC; ++s2) {
      const float inj = round_bf16(combined * gv[s2]);
      res[s2][i] = f32_to_bf16(col(rv[s2]) + inj);
    }
  }
#pragma unroll
  for (int s2 = 0; s2 < HC; ++s2)
    *reinterpret_cast<uint2*>(out + o + size_t(s2) * hidden) =
        make_uint2(uint32_t(res[s2][0]) | (uint32_t(res[s2][1]) << 16),
                   uint32_t(res[s2][2]) | (uint32_t(res[s2][3]) << 16));
}

// moe_reduce_epilogue4_kernel's slot sum and stream write fused with the next
// hyper-connection's norm (hc_norm_kernel's arithmetic, with the operand
// plane): one workgroup per (stream, row) as the norm kernel has, each
// summing the row's slots again for its own stream (K consecutive columns per
// thread); the written stream goes through LDS so that thread t then takes
// columns t + 256 k, and the stream's sum of squares runs over the same
// columns in the same order as the norm kernel's thread t.
// Same bits as the two launches; hc == 4, hidden = 256 K.
template <int K>
__global__ __launch_bounds__(256) void moe_reduce_norm_kernel(
    const uint16_t* __restrict__ p, const uint16_t* __restrict__ factor,
    uint16_t* __restrict__ h, const uint16_t* __restrict__ gate, int top_k,
    const uint16_t* __restrict__ scale, float eps, uint16_t* __restrict__ xn,
    char* __restrict__ plane) {
  constexpr int HC = 4;
  constexpr int hidden = 256 * K;
  constexpr int CPT = K;  // consecutive columns per thread in the slot sum
  __shared__ float red[4];
  __shared__ __align__(16) uint16_t hs_[hidden];  // the written stream
  __shared__ __align__(16) uint16_t ys[hidden];
  const int s = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const uint16_t* pr = p + size_t(row) * (top_k + 1) * hidden;
  uint16_t* hr = h + (size_t(row) * HC + s) * hidden;
  const float f = bf16_to_f32(factor[row]);
  const float gv = bf16_to_f32(gate[size_t(row) * HC + s]);
  const int lanes = top_k < 8 ? top_k : 8;
  // slot sum of columns CPT t .. CPT t + CPT - 1 (every load issued first)
  {
    const int c0 = CPT * t;
    uint16_t pv[kRedMaxK][CPT], sh[CPT], rv[CPT];
    // CPT consecutive bf16 values, as one load when they fill 8 or 16 bytes
    auto load = [&](const uint16_t* src, uint16_t (&dst)[CPT]) {
      if constexpr (CPT == 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dst[2 * i] = uint16_t(w[i]);
          dst[2 * i + 1] = uint16_t(w[i] >> 16);
        }
      } else if constexpr (CPT == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        dst[0] = uint16_t(v.x);
        dst[1] = uint16_t(v.x >> 16);
        dst[2] = uint16_t(v.y);
        dst[3] = uint16_t(v.y >> 16);
      } else {
#pragma unroll
        for (int i = 0; i < CPT; ++i) dst[i] = src[i];
      }
    };
#pragma unroll
    for (int sl = 0; sl < kRedMaxK; ++sl)
      load(pr + size_t(sl < top_k ? sl : top_k) * hidden + c0, pv[sl]);
    load(pr + size_t(top_k) * hidden + c0, sh);
    load(hr + c0, rv);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float acc[8];
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        float v = bf16_to_f32(pv[a][i]);
        if (a + 8 < top_k) v = round_bf16(v + bf16_to_f32(pv[a + 8][i]));
        acc[a] = v;
      }
      float routed = acc[0];
#pragma unroll
      for (int a = 1; a < 8; ++a)
        if (a < lanes) routed = round_bf16(acc[a] + routed);
      routed = round_bf16(routed);
      const float weighted = round_bf16(bf16_to_f32(sh[i]) * f);
      const float combined = round_bf16(routed + weighted);
      const float inj = round_bf16(combined * gv);
      const uint16_t o = f32_to_bf16(bf16_to_f32(rv[i]) + inj);
      hr[c0 + i] = o;
      hs_[c0 + i] = o;
    }
  }
  __syncthreads();
  float xv[K];
#pragma unroll
  for (int k = 0; k < K; ++k) xv[k] = bf16_to_f32(hs_[t + 256 * k]);
  // the stream's norm (hc_norm_kernel<K>'s order)
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) acc = acc + xv[k] * xv[k];
  for (int o = 32; o > 0; o >>= 1) acc = acc + __shfl_xor(acc, o, 64);
  if (lane == 0) red[wave] = acc;
  __syncthreads();
  const float total = ((red[0] + red[1]) + red[2]) + red[3];
  const float inv = 1.0f / __builtin_sqrtf(total / float(hidden) + eps);
  uint16_t* xr = xn + (size_t(row) * HC + s) * hidden;
  const uint16_t* sc = scale + size_t(s) * hidden;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int c = t + 256 * k;
    const uint16_t o = f32_to_bf16((xv[k] * inv) * (bf16_to_f32(sc[c]) + 1.0f));
    xr[c] = o;
    ys[c] = o;
  }
  __syncthreads();
  // the stream's groups of the row's plane (hc_norm_kernel's group split)
  const int kb = lane >> 4;
  constexpr int ng = hidden / xq::kGroup;
  for (int g0 = wave * 16; g0 < ng; g0 += 64) {
    const int gl = g0 + (lane & 15);
    const bool live = gl < ng;
    float fv[16];
    if (live) {
      const uint4 a = *reinterpret_cast<const uint4*>(ys + gl * xq::kGroup + 16 * kb);
      const uint4 b = *reinterpret_cast<const uint4*>(ys + gl * xq::kGroup + 16 * kb + 8);
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        fv[2 * i] = u2f(w[i] << 16);
        fv[2 * i + 1] = u2f(w[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) fv[i] = 0.0f;
    }
    xq::digitize_unit(fv, row, s * ng + gl, kb, live, plane, HC * ng);
  }
}

}  // namespace

int moe_route(const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
              int64_t shared_stride, int rows, int experts, int top_k, uint32_t* ids,
              uint16_t* scores, uint16_t* factor, hipStream_t s) {
  const int per = experts / 64;
#define MX_ROUTE(P)                                                                          \
  case P:                                                                                    \
    hipLaunchKernelGGL(route_kernel<P>, dim3(rows), dim3(64), 0, s, logits, logit_stride,    \
                       shared_logit, shared_stride, experts, top_k, ids, scores, factor);    \
    break;
  switch (per) {
    MX_ROUTE(1) MX_ROUTE(2) MX_ROUTE(4) MX_ROUTE(8) MX_ROUTE(16)
    default: return MX_EUNSUPPORTED;
  }
#undef MX_ROUTE
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}
int moe_route_plan(const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
                   int64_t shared_stride, int rows, int experts, int top_k, uint32_t* ids,
                   uint16_t* scores, uint16_t* factor, MoePlan* plan, hipStream_t s) {
  if (rows > 8) {  // one wave per row: two launches beyond eight rows
    if (int rc = moe_route(logits, logit_stride, shared_logit, shared_stride, rows, experts,
                           top_k, ids, scores, factor, s);
        rc != MX_OK)
      return rc;
    return moe_plan(ids, rows, top_k, plan, s);
  }
  if (rows < 1) return MX_EINVAL;
  const int per = experts / 64;
#define MX_ROUTE(P)                                                                           \
  case P:                                                                                     \
    hipLaunchKernelGGL(route_plan_kernel<P>, dim3(1), dim3(512), 0, s, logits, logit_stride,  \
                       shared_logit, shared_stride, rows, top_k, ids, scores, factor, plan);  \
    break;
  switch (per) {
    MX_ROUTE(1) MX_ROUTE(2) MX_ROUTE(4) MX_ROUTE(8) MX_ROUTE(16)
    default: return MX_EUNSUPPORTED;
  }
#undef MX_ROUTE
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}
int moe_plan(const uint32_t* ids, int rows, int top_k, MoePlan* plan, hipStream_t s) {
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(256), 0, s, ids, rows, top_k, plan);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int chunk_max_items(int rows, int experts, int top_k) {
  // an expert with c routes gives ceil(c / 16) <= 1 + (c - 1) / 16 items
  const int routes = rows * top_k;
  return (routes < experts ? routes : experts) + (routes + 15) / 16 + (rows + 15) / 16;
}

int chunk_plan(const uint32_t* ids, int rows, int experts, int top_k, ChunkPlan* plan,
               hipStream_t s) {
  if (rows < 1 || rows > kPrefillChunk || top_k < 1 || top_k > 16 || experts < 1 ||
      experts > kChunkMaxExperts)
    return MX_EUNSUPPORTED;
  hipLaunchKernelGGL(chunk_plan_kernel, dim3(1), dim3(kChunkPlanThreads), 0, s, ids, rows,
                     experts, top_k, plan);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int moe_gate_up(const uint16_t* x, const MoePlan* plan, int rows, int top_k, const QBank& gate,
                const QBank& up, const QWeight& sgate, const QWeight& sup, uint16_t* h,
                hipStream_t s) {
  const int routes = rows * top_k + 1;
  const int hs = gate.n > sgate.n ? gate.n : sgate.n;  // h row stride (workspace layout)
  // rows per workgroup is fixed by K = hidden, shared by routed and shared experts
  const int L = qmv_lanes_per_row(gate.k);
  const int rows_per_block = kWaves * (64 / L) * kQRows;
  const dim3 grid((hs + rows_per_block - 1) / rows_per_block, routes);
#define MX_GU(B) \
  case B: hipLaunchKernelGGL(gate_up_kernel<B>, grid, dim3(256), 0, s, x, plan, top_k, gate, up, sgate, sup, h, hs); break;
  switch (gate.bits) {
    MX_GU(4) MX_GU(5) MX_GU(6) MX_GU(8)
    default: return MX_EUNSUPPORTED;
  }
#undef MX_GU
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int moe_down(const uint16_t* h, const MoePlan* plan, const uint16_t* scores, int rows, int top_k,
             int inter, int shared_inter, const QBank& down, const QWeight& sdown, uint16_t* p,
             hipStream_t s) {
  const int routes = rows * top_k + 1;
  const int hs = inter > shared_inter ? inter : shared_inter;
  // rows per workgroup shrink as K = inter grows: size the grid for the
  // deeper of the two (workgroups past the end of a shallower route exit)
  const int kmax = down.k > sdown.k ? down.k : sdown.k;
  const int L = qmv_lanes_per_row(kmax);
  const int rows_per_block = kWaves * (64 / L) * kQRows;
  const dim3 grid((down.n + rows_per_block - 1) / rows_per_block, routes);
#define MX_DN(B) \
  case B: hipLaunchKernelGGL(down_kernel<B>, grid, dim3(256), 0, s, h, plan, scores, top_k, down, sdown, p, hs); break;
  switch (down.bits) {
    MX_DN(4) MX_DN(5) MX_DN(6) MX_DN(8)
    default: return MX_EUNSUPPORTED;
  }
#undef MX_DN
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

size_t moe_workspace_bytes(int rows, int top_k, int inter) {
  // h, then the work list: a MoePlan (<= 8 rows) or a ChunkPlan
  const size_t h = size_t(rows) * (top_k + 1) * inter * sizeof(uint16_t);
  return ((h + 255) / 256) * 256 + (rows > 8 ? sizeof(ChunkPlan) : sizeof(MoePlan));
}

int moe_experts(const uint16_t* x, const uint32_t* ids, const uint16_t* scores, int rows,
                int top_k, const QBank& gate, const QBank& up, const QBank& down,
                const QWeight& sgate, const QWeight& sup, const QWeight& sdown, void* workspace,
                uint16_t* p, hipStream_t s) {
  const int inter = gate.n > sgate.n ? gate.n : sgate.n;
  uint16_t* h = static_cast<uint16_t*>(workspace);
  const size_t hb = size_t(rows) * (top_k + 1) * inter * sizeof(uint16_t);
  MoePlan* plan = reinterpret_cast<MoePlan*>(static_cast<char*>(workspace) + ((hb + 255) / 256) * 256);
  int rc = moe_plan(ids, rows, top_k, plan, s);
  if (rc != MX_OK) return rc;
  rc = moe_gate_up(x, plan, rows, top_k, gate, up, sgate, sup, h, s);
  if (rc != MX_OK) return rc;
  return moe_down(h, plan, scores, rows, top_k, gate.n, sgate.n, down, sdown, p, s);
}

int moe_reduce(const uint16_t* p, int rows, int top_k, int hidden, uint16_t* routed,
               hipStream_t s) {
  const dim3 grid((hidden + 255) / 256, rows);
  hipLaunchKernelGGL(moe_reduce_kernel, grid, dim3(256), 0, s, p, top_k, hidden, routed);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int moe_hc_epilogue(const uint16_t* routed, const uint16_t* shared, const uint16_t* factor,
                    const uint16_t* residual, const uint16_t* gate, int rows, int hc, int hidden,
                    uint16_t* out, hipStream_t s) {
  const dim3 grid((hidden + 255) / 256, rows);
  hipLaunchKernelGGL(moe_epilogue_kernel, grid, dim3(256), 0, s, routed, shared, factor, residual,
                     gate, hc, hidden, out);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

bool moe_reduce_norm_supported(int rows, int top_k, int hc, int hidden) {
  return rows >= 1 && rows <= 8 && top_k >= 1 && top_k < kRedMaxK && hc == 4 &&
         hidden % 256 == 0 && hidden / 256 >= 1 && hidden / 256 <= 8;
}

int moe_reduce_norm(const uint16_t* p, const uint16_t* factor, uint16_t* h, const uint16_t* gate,
                    int rows, int top_k, int hc, int hidden, const uint16_t* scale, float eps,
                    uint16_t* xn, char* plane, hipStream_t s) {
  if (!moe_reduce_norm_supported(rows, top_k, hc, hidden)) return MX_EUNSUPPORTED;
  switch (hidden / 256) {
#define MX_RN(KK)                                                                              \
  case KK:                                                                                     \
    hipLaunchKernelGGL(moe_reduce_norm_kernel<KK>, dim3(4, rows), dim3(256), 0, s, p, factor, h, \
                       gate, top_k, scale, eps, xn, plane);                                    \
    break;
    MX_RN(1) MX_RN(2) MX_RN(3) MX_RN(4) MX_RN(5) MX_RN(6) MX_RN(7) MX_RN(8)
#undef MX_RN
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int moe_reduce_hc_epilogue(const uint16_t* p, const uint16_t* factor, const uint16_t* residual,
                           const uint16_t* gate, int rows, int top_k, int hc, int hidden,
                           uint16_t* out, hipStream_t s) {
  if (hc == 4 && top_k < kRedMaxK && hidden % 4 == 0) {
    const dim3 grid4((hidden / 4 + 63) / 64, rows);
    hipLaunchKernelGGL(moe_reduce_epilogue4_kernel, grid4, dim3(64), 0, s, p, factor, residual,
                       gate, top_k, hidden, out);
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
  }
  const dim3 grid((hidden + 255) / 256, rows);
  hipLaunchKernelGGL(moe_reduce_epilogue_kernel, grid, dim3(256), 0, s, p, factor, residual, gate,
                     top_k, hc, hidden, out);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
