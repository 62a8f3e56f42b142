// Hyper-connection input projection on the matrix cores (decode, 1..8 rows):
// grouped RMS norm -> down (low rank + inject rows) -> activation -> up -> mix,
// in two launches (reference HyperConnection::forward_reference,
// src/hybrid.rs:78-99; compiled::activate / injection / mix,
// src/compiled.rs:46-86).
//
//  hc_down_kernel: grid (row groups of 64, S K-slices).  Each K-slice lies in
//    one stream; the workgroup loads that stream of every activation row,
//    forms its RMS norm, stages the normalised slice (written out as xn by row
//    group 0, for the mix) and streams 4 tiles of down rows over it, writing
//    fp32 partial sums part[slice][m][row].
//  hc_up_kernel: grid (16-column groups).  Every workgroup adds the S partials
//    of all down rows in slice order, applies the activation in registers
//    (low-rank rows -> silu(v / hc) into the MFMA staging; inject rows ->
//    2 sigmoid(v / hc), written by group 0), then streams the 4 stream tiles of
//    up rows and mixes: mixed[c] = mean_s sigmoid(p_s) * xn_s[c].
//
// Arithmetic: matrix-core sums (skinny_core.hpp) and the element-wise steps of
// the exact kernels (bf16 rounding per operation); results agree with the
// exact path within summation-order tolerance.
#include "common.hpp"
#include "kernels.hpp"
#include "skinny_core.hpp"

namespace mx {

namespace {

constexpr int kSlices = 8;

__device__ __forceinline__ float sigmoid_bf16(float x) {
  const float e = round_bf16(expf_(__builtin_fabsf(x)));
  const float d = round_bf16(1.0f + e);
  const float y = round_bf16(1.0f / d);
  return x < 0.0f ? y : round_bf16(1.0f - y);
}

// Writes one staged 8-value unit (value v of row m, unit u of the slice) in
// operand order, and its group sum when this lane leads its group of 8 lanes.
__device__ __forceinline__ void stage_unit(char* lds, int steps, uint4 val, int m, int u,
                                           bool live) {
  uint4* xs = reinterpret_cast<uint4*>(lds);
  float* sx = reinterpret_cast<float*>(lds + steps * sk::kStepBytes + sk::kZeroBytes);
  const uint32_t d[4] = {val.x, val.y, val.z, val.w};
  float sum = 0.0f;
#pragma unroll
  for (int h = 0; h < 4; ++h) sum = sum + u2f(d[h] << 16) + u2f(d[h] & 0xffff0000u);
  sum = sum + __shfl_xor(sum, 1, 64);
  sum = sum + __shfl_xor(sum, 2, 64);
  sum = sum + __shfl_xor(sum, 4, 64);
  if (live) {
    if ((u & 7) == 0) sx[(u >> 3) * 8 + m] = sum;
    const int s = u >> 4, o = u & 15;
    xs[(s * 4 + (o & 3)) * 32 + (o >> 2) * 8 + m] = sk::permute_x(val);
  }
}

__device__ __forceinline__ void zero_block(char* lds, int steps, int nthreads) {
  uint2* zero = reinterpret_cast<uint2*>(lds + steps * sk::kStepBytes);
  for (int t = threadIdx.x; t < sk::kZeroBytes / 8; t += nthreads) zero[t] = make_uint2(0, 0);
}

// ---------------------------------------------------------------------------
// hidden <= 2048 and hidden % (kSlices / hc * 128) == 0 (checked on the host).
template <int BITS>
__global__ __launch_bounds__(256) void hc_down_kernel(QWeight w, const uint16_t* __restrict__ h,
                                                      const uint16_t* __restrict__ scale, int M,
                                                      int hidden, int hc, float eps,
                                                      uint16_t* __restrict__ xn,
                                                      float* __restrict__ part, int npad) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float ssq[4][8];
  const int tg = blockIdx.x, slice = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;
  const int K = w.k;                     // hc * hidden
  const int slen = K / kSlices;          // values per slice
  const int stream = (slice * slen) / hidden;
  const int sstart = slice * slen - stream * hidden;  // slice offset within the stream
  const int steps = slen / sk::kSuper;
  const int ks0 = slice * steps;
  const int n = w.n, G = K >> 6;
  const int row = min(tg * 64 + wave * 16 + j, n - 1);
  // stream rows: M x hidden values, units of 8; thread t holds unit t + 256 k
  const int units = hidden / 8;          // per row
  const int total = M * units;
  constexpr int PER = 8;                 // 8 rows x 2048 / 8 / 256
  uint4 v[PER];
  uint4 sc[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = min(int(threadIdx.x) + k * 256, total - 1);
    const int m = i / units, u = i - m * units;
    v[k] = *reinterpret_cast<const uint4*>(h + size_t(m) * K + size_t(stream) * hidden + u * 8);
    sc[k] = *reinterpret_cast<const uint4*>(scale + size_t(stream) * hidden + u * 8);
  }
  const sk::DenseRows none{h, 0, 1};
  sk::Stream<BITS, false, sk::DenseRows, 8> st(w.codes + size_t(row) * (size_t(K) * BITS / 32),
                                               w.scales + size_t(row) * G,
                                               w.biases + size_t(row) * G, K / sk::kSuper, ks0,
                                               steps, ks0, lds,
                                               reinterpret_cast<const float*>(
                                                   lds + steps * sk::kStepBytes + sk::kZeroBytes),
                                               none, 1);
  st.prefetch();
  // sums of squares per row (thread order, then waves 0..3)
  float acc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = 0.0f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = int(threadIdx.x) + k * 256;
    if (i < total) {
      const int m = i / units;
      const uint32_t d[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
      float s2 = 0.0f;
#pragma unroll
      for (int hh = 0; hh < 4; ++hh) {
        const float a = u2f(d[hh] << 16), b = u2f(d[hh] & 0xffff0000u);
        s2 = s2 + a * a + b * b;
      }
#pragma unroll
      for (int mm = 0; mm < 8; ++mm)
        if (mm == m) acc[mm] = acc[mm] + s2;
    }
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    float a = acc[m];
    for (int o = 32; o > 0; o >>= 1) a = a + __shfl_xor(a, o, 64);
    if (lane == 0) ssq[wave][m] = a;
  }
  zero_block(lds, steps, 256);
  __syncthreads();
  // normalised slice values, staged (and written out by row group 0)
  const int sunits = slen / 8;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = int(threadIdx.x) + k * 256;
    const int ic = min(i, total - 1);
    const int m = ic / units, u = ic - m * units;
    const int su = u - sstart / 8;  // unit within the slice
    const bool in_slice = i < total && su >= 0 && su < sunits;
    const float tot = ((ssq[0][m] + ssq[1][m]) + ssq[2][m]) + ssq[3][m];
    const float inv = 1.0f / __builtin_sqrtf(tot / float(hidden) + eps);
    const uint32_t d[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
    const uint32_t e[4] = {sc[k].x, sc[k].y, sc[k].z, sc[k].w};
    uint32_t o[4];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      const float a = u2f(d[hh] << 16), b = u2f(d[hh] & 0xffff0000u);
      const float ea = u2f(e[hh] << 16), eb = u2f(e[hh] & 0xffff0000u);
      const uint32_t ya = f32_to_bf16((a * inv) * (ea + 1.0f));
      const uint32_t yb = f32_to_bf16((b * inv) * (eb + 1.0f));
      o[hh] = ya | (yb << 16);
    }
    const uint4 val = make_uint4(o[0], o[1], o[2], o[3]);
    // every lane of a wave takes part in the group-sum shuffles; only slice
    // units are stored (a group of 8 lanes is wholly inside or outside)
    if ((k * 256 + int(threadIdx.x & ~63)) < total)
      stage_unit(lds, steps, val, m, su < 0 ? 0 : su, in_slice);
    if (in_slice && tg == 0)
      *reinterpret_cast<uint4*>(xn + size_t(m) * K + size_t(stream) * hidden + u * 8) = val;
  }
  // rows M..7 of the slice are zero
  {
    uint4* xs = reinterpret_cast<uint4*>(lds);
    float* sxp = reinterpret_cast<float*>(lds + steps * sk::kStepBytes + sk::kZeroBytes);
    for (int i = threadIdx.x; i < (8 - M) * sunits; i += 256) {
      const int m = M + i / sunits, u = i % sunits;
      const int s = u >> 4, o = u & 15;
      xs[(s * 4 + (o & 3)) * 32 + (o >> 2) * 8 + m] = make_uint4(0, 0, 0, 0);
      if ((u & 7) == 0) sxp[(u >> 3) * 8 + m] = 0.0f;
    }
  }
  __syncthreads();
  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  st.run(steps * sk::kStepBytes, y);
  sk::join_parities(y);
  const int r = tg * 64 + wave * 16 + j;
  if (q < 2 && r < n) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) part[(size_t(slice) * 8 + 4 * q + rr) * npad + r] = y[rr];
  }
}

// ---------------------------------------------------------------------------
// n_down = rank (+ hc inject rows); rank % 256 == 0 is not required, but
// rank <= 512 and rank % 128 == 0 (checked on the host).
template <int BITS>
__global__ __launch_bounds__(1024) void hc_up_kernel(QWeight up, const float* __restrict__ part,
                                                     int npad, int n_down, int rank, int M,
                                                     int hidden, int hc,
                                                     const uint16_t* __restrict__ xn,
                                                     uint16_t* __restrict__ mixed,
                                                     uint16_t* __restrict__ inj) {
  extern __shared__ __align__(16) char lds[];
  __shared__ __align__(16) uint16_t lo[8 * 512];
  __shared__ float yt[8 * 64];
  const int tg = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15;
  const int steps = rank / sk::kSuper;
  const int G = rank >> 6;
  // the up tiles (waves 0..3: stream t) prefetch their weights first
  const int t = wave & 3;
  const int urow = t * hidden + min(tg * 16 + j, hidden - 1);
  const sk::DenseRows none{mixed, 0, 1};
  sk::Stream<BITS, false, sk::DenseRows, 4, 8> st(
      up.codes + size_t(urow) * (size_t(rank) * BITS / 32), up.scales + size_t(urow) * G,
      up.biases + size_t(urow) * G, steps, 0, steps, 0, lds,
      reinterpret_cast<const float*>(lds + steps * sk::kStepBytes + sk::kZeroBytes), none, 1);
  if (wave < 4) st.prefetch();
  // 1. partial sums -> activation (quads of 4 down rows per thread)
  const int quads = npad / 4;
  if (int(threadIdx.x) < 8 * quads) {
    const int m = threadIdx.x / quads, qd = threadIdx.x - m * quads;
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 pv[kSlices];
#pragma unroll
    for (int i = 0; i < kSlices; ++i)
      pv[i] = *reinterpret_cast<const float4*>(part + (size_t(i) * 8 + m) * npad + 4 * qd);
#pragma unroll
    for (int i = 0; i < kSlices; ++i) {
      s.x = s.x + pv[i].x;
      s.y = s.y + pv[i].y;
      s.z = s.z + pv[i].z;
      s.w = s.w + pv[i].w;
    }
    const float vals[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 4 * qd + k;
      if (r >= n_down) continue;
      const float tt = round_bf16(round_bf16(vals[k]) / float(hc));
      if (r < rank) {
        lo[m * rank + r] = m < M ? f32_to_bf16(tt * sigmoid_bf16(tt)) : uint16_t(0);
      } else if (inj && tg == 0 && m < M) {
        inj[size_t(m) * hc + (r - rank)] = f32_to_bf16(sigmoid_bf16(tt) * 2.0f);
      }
    }
  }
  zero_block(lds, steps, 1024);
  __syncthreads();
  // 2. stage lo (8 rows x rank) in operand order with its group sums
  {
    const int units = rank / 8;
    const int i = threadIdx.x;  // 8 * units <= 512 <= 1024 threads
    const bool live = i < 8 * units;
    const int ic = live ? i : 0;
    const int m = ic / units, u = ic - m * units;
    const uint4 val = *reinterpret_cast<const uint4*>(lo + m * rank + u * 8);
    if (int(threadIdx.x & ~63) < 8 * units) stage_unit(lds, steps, val, m, u, live);
  }
  __syncthreads();
  // 3. up tiles (waves 0..3) and the mix
  if (wave < 4) {
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    st.run(steps * sk::kStepBytes, y);
    sk::join_parities(y);
    const int q = lane >> 4;
    if (q < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) yt[(4 * q + r) * 64 + t * 16 + j] = y[r];
    }
  }
  __syncthreads();
  if (threadIdx.x >= 128) return;
  const int m = threadIdx.x >> 4, cj = threadIdx.x & 15;
  const int c = tg * 16 + cj;
  if (m >= M || c >= hidden) return;
  float sum = 0.0f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float p = round_bf16(yt[m * 64 + s * 16 + cj]);
    const float x = bf16_to_f32(xn[size_t(m) * hc * hidden + size_t(s) * hidden + c]);
    sum = sum + round_bf16(sigmoid_bf16(p) * x);
  }
  mixed[size_t(m) * hidden + c] = f32_to_bf16(round_bf16(sum) / 4.0f);
}

}  // namespace

int hc_fused_npad(int n_down) { return ((n_down + 63) / 64) * 64; }
size_t hc_fused_part_bytes(int n_down) {
  return size_t(kSlices) * 8 * hc_fused_npad(n_down) * sizeof(float);
}

bool hc_fused_supported(const QWeight& down, const QWeight& up, int hc, int hidden, int rank) {
  const int slen = down.k / kSlices;
  return hc == 4 && down.k == hc * hidden && hidden <= 2048 && slen % sk::kSuper == 0 &&
         hidden % slen == 0 && down.group_size == 64 && up.group_size == 64 &&
         down.k % 512 == 0 && down.bits == up.bits && up.k == rank && up.n == hc * hidden &&
         rank % sk::kSuper == 0 && rank <= 512 && (rank % 512 == 0 || rank <= 1024) &&
         rank % 256 == 0 && hc_fused_npad(down.n) * 2 <= 1024 &&
         (down.bits == 4 || down.bits == 5 || down.bits == 6 || down.bits == 8);
}

int hc_fused(const QWeight& down, const QWeight& up, const uint16_t* h, const uint16_t* scale,
             int M, int hc, int hidden, int rank, float eps, uint16_t* xn, float* part,
             uint16_t* mixed, uint16_t* inj, hipStream_t s) {
  if (M < 1 || M > 8 || !hc_fused_supported(down, up, hc, hidden, rank)) return MX_EUNSUPPORTED;
  const int npad = hc_fused_npad(down.n);
  const int steps = down.k / kSlices / sk::kSuper;
  const dim3 g1((down.n + 63) / 64, kSlices);
  const int lb1 = sk::stage_bytes(steps);
  const int lb2 = sk::stage_bytes(rank / sk::kSuper);
  switch (down.bits) {
#define MX_HC(B)                                                                               \
  case B:                                                                                      \
    hipLaunchKernelGGL(hc_down_kernel<B>, g1, dim3(256), lb1, s, down, h, scale, M, hidden, hc, \
                       eps, xn, part, npad);                                                   \
    hipLaunchKernelGGL(hc_up_kernel<B>, dim3((hidden + 15) / 16), dim3(1024), lb2, s, up, part, \
                       npad, down.n, rank, M, hidden, hc, xn, mixed, inj);                     \
    break;
    MX_HC(4) MX_HC(5) MX_HC(6) MX_HC(8)
#undef MX_HC
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
