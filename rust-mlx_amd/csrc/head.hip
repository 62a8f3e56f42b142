// Greedy vocabulary head for gfx950: quantised head projection fused with a
// per-workgroup argmax of the bf16-rounded logits, then a cross-workgroup
// argmax reduction.  Logits never reach HBM.
//
// Reference: greedy_head::project (src/greedy_head.rs:40-126),
// kernels/greedy_head.metal (per-block best of bf16(logit), lowest id on ties)
// and kernels/greedy_reduce.metal (argmax of the partials; NaN never wins).
// The default reference path, argmax_axis(head.forward_rows(x))
// (src/bin/batch-bench.rs:118-120), selects the same token: the selection
// rule below is a total order, so the split into partials cannot change it.
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"
#include "qmv_core.hpp"

namespace mx {

namespace {

constexpr int kWaves = 4;

// Argmax update: larger value wins; equal values keep the lower id; NaN never
// compares greater, so it never wins.
__device__ __forceinline__ void better(float v, uint32_t id, float& best, uint32_t& best_id) {
  if (v > best || (v == best && id < best_id)) {
    best = v;
    best_id = id;
  }
}

__device__ __forceinline__ void wave_best(float& best, uint32_t& best_id) {
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(best, o, 64);
    const uint32_t id = uint32_t(__shfl_xor(int(best_id), o, 64));
    better(v, id, best, best_id);
  }
}

template <int BITS, int M>
__global__ __launch_bounds__(256) void head_kernel(const uint32_t* __restrict__ codes,
                                                   const uint16_t* __restrict__ scales,
                                                   const uint16_t* __restrict__ biases,
                                                   const uint16_t* __restrict__ x, int n, int k,
                                                   int gs, int L, int parts,
                                                   float* __restrict__ maxima,
                                                   uint32_t* __restrict__ indices) {
  __shared__ float bv[kWaves][M];
  __shared__ uint32_t bi[kWaves][M];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & (L - 1);
  const int lg = lane / L;
  const int row0 = ((blockIdx.x * kWaves + wave) * (64 / L) + lg) * kQRows;
  float best[M];
  uint32_t best_id[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    best[m] = u2f(0xff800000u);
    best_id[m] = 0xffffffffu;
  }
  if (row0 < n) {
    int rows[kQRows];
#pragma unroll
    for (int r = 0; r < kQRows; ++r) rows[r] = min(row0 + r, n - 1);
    const uint16_t* xrow[M];
#pragma unroll
    for (int m = 0; m < M; ++m) xrow[m] = x + size_t(m) * k;
    float out[M][kQRows];
    qmv_core<BITS, M>(codes, scales, biases, k, gs, xrow, rows, li, L, out);
#pragma unroll
    for (int r = 0; r < kQRows; ++r)
      if (row0 + r < n)
#pragma unroll
        for (int m = 0; m < M; ++m) better(round_bf16(out[m][r]), uint32_t(row0 + r), best[m], best_id[m]);
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    wave_best(best[m], best_id[m]);
    if (lane == 0) {
      bv[wave][m] = best[m];
      bi[wave][m] = best_id[m];
    }
  }
  __syncthreads();
  if (threadIdx.x < M) {
    const int m = threadIdx.x;
    float b = bv[0][m];
    uint32_t id = bi[0][m];
    for (int w = 1; w < kWaves; ++w) better(bv[w][m], bi[w][m], b, id);
    maxima[size_t(m) * parts + blockIdx.x] = b;
    indices[size_t(m) * parts + blockIdx.x] = id;
  }
}

// One workgroup per row: the best (value, id) over `parts` partials.  A row
// whose partials are all -inf or NaN selects id 0 (MLX argmax convention).
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ maxima,
                                                     const uint32_t* __restrict__ indices,
                                                     int parts, uint32_t* __restrict__ tokens) {
  __shared__ float bv[4];
  __shared__ uint32_t bi[4];
  const int row = blockIdx.x;
  float best = u2f(0xff800000u);
  uint32_t best_id = 0;
  for (int j = threadIdx.x; j < parts; j += 256)
    better(maxima[size_t(row) * parts + j], indices[size_t(row) * parts + j], best, best_id);
  wave_best(best, best_id);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bv[wave] = best;
    bi[wave] = best_id;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) better(bv[w], bi[w], bv[0], bi[0]);
    tokens[row] = bi[0];
  }
}

// argmax over bf16 logits [rows, n] (the reference's default head path).
__global__ __launch_bounds__(256) void argmax_bf16_kernel(const uint16_t* __restrict__ logits,
                                                          int n, uint32_t* __restrict__ tokens) {
  __shared__ float bv[4];
  __shared__ uint32_t bi[4];
  const int row = blockIdx.x;
  float best = u2f(0xff800000u);
  uint32_t best_id = 0;
  for (int j = threadIdx.x; j < n; j += 256)
    better(bf16_to_f32(logits[size_t(row) * n + j]), uint32_t(j), best, best_id);
  wave_best(best, best_id);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bv[wave] = best;
    bi[wave] = best_id;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) better(bv[w], bi[w], bv[0], bi[0]);
    tokens[row] = bi[0];
  }
}

template <int BITS, int M>
void launch_head(const QWeight& w, const uint16_t* x, float* maxima, uint32_t* indices, int parts,
                 hipStream_t s) {
  const int L = qmv_lanes_per_row(w.k);
  hipLaunchKernelGGL((head_kernel<BITS, M>), dim3(parts), dim3(64 * kWaves), 0, s, w.codes,
                     w.scales, w.biases, x, w.n, w.k, w.group_size, L, parts, maxima, indices);
}

template <int BITS>
void head_m(const QWeight& w, const uint16_t* x, int m, float* maxima, uint32_t* indices,
            int parts, hipStream_t s) {
  switch (m) {
    case 1: launch_head<BITS, 1>(w, x, maxima, indices, parts, s); break;
    case 2: launch_head<BITS, 2>(w, x, maxima, indices, parts, s); break;
    case 3: launch_head<BITS, 3>(w, x, maxima, indices, parts, s); break;
    case 4: launch_head<BITS, 4>(w, x, maxima, indices, parts, s); break;
    case 5: launch_head<BITS, 5>(w, x, maxima, indices, parts, s); break;
    case 6: launch_head<BITS, 6>(w, x, maxima, indices, parts, s); break;
    case 7: launch_head<BITS, 7>(w, x, maxima, indices, parts, s); break;
    default: launch_head<BITS, 8>(w, x, maxima, indices, parts, s); break;
  }
}

}  // namespace

// Number of partials per row for a head of n rows and depth k.
int head_parts(int n, int k) {
  const int L = qmv_lanes_per_row(k);
  const int rows_per_block = kWaves * (64 / L) * kQRows;
  return (n + rows_per_block - 1) / rows_per_block;
}

int head_partials(const QWeight& w, const uint16_t* x, int m, float* maxima, uint32_t* indices,
                  int* parts_out, hipStream_t s) {
  const int parts = head_parts(w.n, w.k);
  *parts_out = parts;
  switch (w.bits) {
    case 4: head_m<4>(w, x, m, maxima, indices, parts, s); break;
    case 5: head_m<5>(w, x, m, maxima, indices, parts, s); break;
    case 6: head_m<6>(w, x, m, maxima, indices, parts, s); break;
    case 8: head_m<8>(w, x, m, maxima, indices, parts, s); break;
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int argmax_reduce(const float* maxima, const uint32_t* indices, int rows, int parts,
                  uint32_t* tokens, hipStream_t s) {
  hipLaunchKernelGGL(reduce_kernel, dim3(rows), dim3(256), 0, s, maxima, indices, parts, tokens);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

// Partials of head_argmax_noalloc: a file-scope device array, one copy per
// GPU, shared by every call on that GPU (calls that overlap on one GPU race).
// Host code never passes `scratch` itself to a kernel: in host code the name
// stands for a host-side shadow, so kernels receive the device address that
// hipGetSymbolAddress returns for the current device.
namespace {
__device__ __align__(256) unsigned char scratch[kHeadNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};
}  // namespace

// The current device's copy of `scratch`: looked up on the first call on each
// device (with that device current) and kept.
static int noalloc_scratch(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MX_EHIP;
  if (dev < 0 || dev >= kMaxDevices) return MX_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return MX_EHIP;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return MX_OK;
}

size_t head_noalloc_bytes(int n, int k, int m) {
  return size_t(head_parts(n, k)) * size_t(m) * (sizeof(float) + sizeof(uint32_t));
}

// head_partials + argmax_reduce with the partials in this device's `scratch`
// instead of a workspace.  Every partial the reduction reads is written by
// the partials launch of the same call, so nothing needs clearing.
int head_argmax_noalloc(const QWeight& w, const uint16_t* x, int m, uint32_t* tokens,
                        hipStream_t s) {
  if (head_noalloc_bytes(w.n, w.k, m) > kHeadNoAllocScratchBytes) return MX_EUNSUPPORTED;
  void* base = nullptr;
  if (int rc = noalloc_scratch(&base); rc != MX_OK) return rc;
  const int parts = head_parts(w.n, w.k);
  float* maxima = static_cast<float*>(base);
  uint32_t* indices = reinterpret_cast<uint32_t*>(maxima + size_t(parts) * m);
  int got = 0;
  if (int rc = head_partials(w, x, m, maxima, indices, &got, s); rc != MX_OK) return rc;
  return argmax_reduce(maxima, indices, m, parts, tokens, s);
}

int argmax_bf16(const uint16_t* logits, int rows, int n, uint32_t* tokens, hipStream_t s) {
  hipLaunchKernelGGL(argmax_bf16_kernel, dim3(rows), dim3(256), 0, s, logits, n, tokens);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
