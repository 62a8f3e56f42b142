// Hyper-connection input projection on the matrix cores (decode, 1..8 rows):
// per-stream RMS norm -> down (low rank + inject rows) -> activation -> up ->
// mix, in two launches (reference HyperConnection::forward_reference,
// src/hybrid.rs:78-99; compiled::activate / injection / mix,
// src/compiled.rs:46-86).
//
// The norm is a per-(row, stream) factor, so it is taken out of the down
// projection: for down row r and activation row m
//   down[m, r] = sum_s inv[m, s] * sum_{k in stream s} W[r, k] * bf16(h[m, k] (w[k] + 1))
// with inv[m, s] = 1 / sqrt(mean_{k in s} h[m, k]^2 + eps).
//
//  hc_down_kernel: grid (16-row tiles of the down matrix, streams).  Each of
//    the workgroup's waves takes SPW super-steps (128 values) of the stream and
//    builds its matrix-core A operands in registers straight from h and the
//    norm weights (no LDS staging, no barrier before the products); the same
//    operands give the group sums of x (an MFMA against ones) and the sums of
//    squares of h (the diagonal of H H^T, one more MFMA).  The waves' partial
//    sums are added in LDS in wave order and written as part[stream][m][row];
//    the tile-0 workgroup of each stream also writes the stream's sums of
//    squares.
//  hc_up_kernel: grid (16-column groups).  Every workgroup forms inv, adds the
//    stream partials of all down rows weighted by inv (stream order), applies
//    the activation (low-rank rows -> silu(v / hc) into the MFMA staging;
//    inject rows -> 2 sigmoid(v / hc), written by group 0; sigmoid and the
//    norm factor from the hardware exp2 / reciprocal / rsqrt), streams the 4
//    stream tiles of up rows, and mixes:
//      mixed[c] = mean_s sigmoid(p_s) * bf16((h_s[c] inv_s) (w_s[c] + 1)).
//
// Arithmetic: matrix-core sums (skinny_core.hpp) in another order than the
// exact kernels; results agree with the exact path within summation-order
// tolerance.
#include "common.hpp"
#include "kernels.hpp"
#include "skinny_core.hpp"

namespace mx {

namespace {

constexpr int kMaxDownWaves = 8;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// sigmoid with the hardware exp2 and reciprocal (about 1 ulp; fast mode).
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// Two fp32 values -> packed bf16 pair (round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// A operand of one MFMA step: bf16(h * (w + 1)) for 8 values, in operand order.
__device__ __forceinline__ uint4 scaled_operand(const uint4& hv, const uint4& wv) {
  const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
  const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = u2f(hw[i] << 16) * (u2f(ww[i] << 16) + 1.0f);
    const float b = u2f(hw[i] & 0xffff0000u) * (u2f(ww[i] & 0xffff0000u) + 1.0f);
    o[i] = pack_bf16(a, b);
  }
  return sk::permute_x(make_uint4(o[0], o[1], o[2], o[3]));
}

// Writes one staged 8-value unit (value unit u of row m) in operand order, and
// its group sum when this lane leads its group.  The lanes of a wave hold unit
// u = (lane / 8) + 8 c of row m = lane % 8: the eight units of a group lie 8
// lanes apart, and consecutive lanes write different rows (no LDS bank
// conflicts).  All 64 lanes take part in the shuffles.
__device__ __forceinline__ void stage_unit(char* lds, int steps, uint4 val, int m, int u) {
  uint4* xs = reinterpret_cast<uint4*>(lds);
  float* sx = reinterpret_cast<float*>(lds + steps * sk::kStepBytes + sk::kZeroBytes);
  const uint32_t d[4] = {val.x, val.y, val.z, val.w};
  float sum = 0.0f;
#pragma unroll
  for (int h = 0; h < 4; ++h) sum = sum + u2f(d[h] << 16) + u2f(d[h] & 0xffff0000u);
  sum = sum + __shfl_xor(sum, 8, 64);
  sum = sum + __shfl_xor(sum, 16, 64);
  sum = sum + __shfl_xor(sum, 32, 64);
  if ((u & 7) == 0) sx[(u >> 3) * 8 + m] = sum;
  const int s = u >> 4, o = u & 15;
  xs[(s * 4 + (o & 3)) * 32 + (o >> 2) * 8 + m] = sk::permute_x(val);
}

__device__ __forceinline__ void zero_block(char* lds, int steps, int nthreads) {
  uint2* zero = reinterpret_cast<uint2*>(lds + steps * sk::kStepBytes);
  for (int t = threadIdx.x; t < sk::kZeroBytes / 8; t += nthreads) zero[t] = make_uint2(0, 0);
}

// ---------------------------------------------------------------------------
// Block: (hidden / 128) / SPW waves (<= kMaxDownWaves).  Lane l = 16 q + j:
// weight row j of the tile; A row j (activation m = j % 8) when the lane is
// live for its group parity (j < 8 == q < 2), values 32 q .. +31 of the
// super-step.
template <int BITS, int SPW>
__global__ __launch_bounds__(64 * kMaxDownWaves) void hc_down_kernel(
    QWeight w, const uint16_t* __restrict__ h, const uint16_t* __restrict__ scale, int M,
    int hidden, float* __restrict__ part, float* __restrict__ ssq, int npad) {
  __shared__ float red[kMaxDownWaves][8][16];
  __shared__ float sred[kMaxDownWaves][8];
  const int tile = blockIdx.x, stream = blockIdx.y;
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;
  const int K = w.k, n = w.n, G = K >> 6;
  const int row = min(tile * 16 + j, n - 1);
  const int ks0 = stream * (hidden / sk::kSuper) + wave * SPW;  // super-step within K
  const int m = j & 7;
  const bool live = ((j < 8) == (q < 2)) && m < M;
  // the lane's data at super-step ks0; super-step ks0 + i sits a constant
  // offset further
  const uint16_t* hrow = h + size_t(m < M ? m : M - 1) * K + size_t(ks0) * sk::kSuper + 32 * q;
  const uint16_t* wrow = scale + size_t(ks0) * sk::kSuper + 32 * q;
  const uint32_t* clane =
      w.codes + size_t(row) * (size_t(K) * BITS / 32) + size_t(4 * BITS) * ks0 + BITS * q;
  const uint16_t* srow = w.scales + size_t(row) * G + 2 * ks0;
  const uint16_t* brow = w.biases + size_t(row) * G + 2 * ks0;
  // every load up front: codes, scale/bias words, h and norm weights
  uint32_t wc[SPW][BITS];
  uint32_t sw[SPW], bw[SPW];
  uint4 hx[SPW][4], wx[SPW][4];
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    sk::load_codes<BITS>(clane, i, wc[i]);
    sw[i] = *reinterpret_cast<const uint32_t*>(srow + 2 * i);
    bw[i] = *reinterpret_cast<const uint32_t*>(brow + 2 * i);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      hx[i][u] = *reinterpret_cast<const uint4*>(hrow + i * sk::kSuper + 8 * u);
      wx[i][u] = *reinterpret_cast<const uint4*>(wrow + i * sk::kSuper + 8 * u);
    }
  }
  const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  const float off = sk::code_offset<BITS>();
  const int hi = q >> 1;
  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  sk::floatx4_t sq = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    uint4 a[4];
    sk::floatx4_t sa = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // select the input, then convert unconditionally (a select, not a branch)
      const uint4 raw = live ? hx[i][u] : zero;
      sq = sk::mfma(raw, raw, sq);
      a[u] = scaled_operand(raw, wx[i][u]);
      sa = sk::mfma(a[u], ones, sa);
    }
    sk::floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = sk::mfma(a[0], sk::b_operand<BITS, 0>(wc[i]), acc);
    acc = sk::mfma(a[1], sk::b_operand<BITS, 1>(wc[i]), acc);
    acc = sk::mfma(a[2], sk::b_operand<BITS, 2>(wc[i]), acc);
    acc = sk::mfma(a[3], sk::b_operand<BITS, 3>(wc[i]), acc);
    const float sc = u2f(hi ? (sw[i] & 0xffff0000u) : (sw[i] << 16));
    const float bi = fmaf_(-off, sc, u2f(hi ? (bw[i] & 0xffff0000u) : (bw[i] << 16)));
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = fmaf_(sc, acc[r], fmaf_(bi, sa[r], y[r]));
  }
  sk::join_parities(y);
  if (q < 2) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * q + r][j] = y[r];
  }
  // sum of squares of row m: D[m][m] + D[m+8][m+8] of H H^T, held by lanes
  // 16 (m / 4) + m and 16 (m / 4) + m + 40, element m % 4
  const int e = j & 3;
  const float dg = e == 0 ? sq[0] : e == 1 ? sq[1] : e == 2 ? sq[2] : sq[3];
  const float dg2 = __shfl(dg, (lane + 40) & 63, 64);
  if (j < 8 && q == (j >> 2)) sred[wave][j] = dg + dg2;
  __syncthreads();
  if (threadIdx.x < 128) {
    const int mm = threadIdx.x >> 4, jj = threadIdx.x & 15;
    float v = red[0][mm][jj];
    for (int wv = 1; wv < waves; ++wv) v = v + red[wv][mm][jj];
    const int r = tile * 16 + jj;
    if (r < n) part[(size_t(stream) * 8 + mm) * npad + r] = v;
    if (tile == 0 && jj == 0) {
      float s2 = sred[0][mm];
      for (int wv = 1; wv < waves; ++wv) s2 = s2 + sred[wv][mm];
      ssq[stream * 8 + mm] = s2;
    }
  }
}

// ---------------------------------------------------------------------------
// n_down = rank (+ hc inject rows); rank = 128 STEPS with STEPS 2 or 4.
// hc == 4.
template <int BITS, int STEPS>
__global__ __launch_bounds__(1024) void hc_up_kernel(QWeight up, const float* __restrict__ part,
                                                     const float* __restrict__ ssq, int npad,
                                                     int n_down, int rank, int M, int hidden,
                                                     float eps, const uint16_t* __restrict__ h,
                                                     const uint16_t* __restrict__ scale,
                                                     uint16_t* __restrict__ mixed,
                                                     uint16_t* __restrict__ inj) {
  constexpr int HC = 4;
  extern __shared__ __align__(16) char lds[];
  __shared__ __align__(16) uint16_t lo[8 * 512];
  __shared__ float yt[8 * 64];
  const int tg = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15;
  constexpr int steps = STEPS;
  const int G = rank >> 6;
  const int K = HC * hidden;
  // 1. stream partials -> down outputs -> activation, one quad of 4 down rows
  //    per thread (8 * npad / 4 <= 1024); the partial loads go out first
  const int quads = npad / 4;
  const int qi = min(int(threadIdx.x), 8 * quads - 1);
  const int qm = qi / quads, qd = qi - qm * quads;
  float4 pv[HC];
  float sv[HC];
#pragma unroll
  for (int s = 0; s < HC; ++s) {
    pv[s] = *reinterpret_cast<const float4*>(part + (size_t(s) * 8 + qm) * npad + 4 * qd);
    sv[s] = ssq[s * 8 + qm];
  }
  // the up tiles (waves 0..3: stream t) prefetch their weights
  const int t = wave & 3;
  const int urow = t * hidden + min(tg * 16 + j, hidden - 1);
  const sk::DenseRows none{mixed, 0, 1};
  sk::Stream<BITS, false, sk::DenseRows, 4, 8> st(
      up.codes + size_t(urow) * (size_t(rank) * BITS / 32), up.scales + size_t(urow) * G,
      up.biases + size_t(urow) * G, steps, 0, steps, 0, lds,
      reinterpret_cast<const float*>(lds + steps * sk::kStepBytes + sk::kZeroBytes), none, 1);
  if (wave < 4) st.prefetch();
  // the mix inputs of this thread (threads < 128: row mm, column c)
  const int mm = (threadIdx.x >> 4) & 7, cj = threadIdx.x & 15;
  const int c = min(tg * 16 + cj, hidden - 1);
  uint16_t hv[HC], wv[HC];
  if (threadIdx.x < 128) {  // waves 0 and 1
#pragma unroll
    for (int s = 0; s < HC; ++s) {
      hv[s] = h[size_t(mm < M ? mm : M - 1) * K + size_t(s) * hidden + c];
      wv[s] = scale[size_t(s) * hidden + c];
    }
  }
  const float inv_hidden = 1.0f / float(hidden);
  if (int(threadIdx.x) < 8 * quads) {
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int s = 0; s < HC; ++s) {
      const float inv = __builtin_amdgcn_rsqf(fmaf_(sv[s], inv_hidden, eps));
      acc.x = fmaf_(inv, pv[s].x, acc.x);
      acc.y = fmaf_(inv, pv[s].y, acc.y);
      acc.z = fmaf_(inv, pv[s].z, acc.z);
      acc.w = fmaf_(inv, pv[s].w, acc.w);
    }
    const float vals[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 4 * qd + k;
      if (r >= n_down) continue;
      const float tt = round_bf16(round_bf16(vals[k]) * (1.0f / HC));
      if (r < rank) {
        lo[qm * rank + r] = qm < M ? f32_to_bf16(tt * sigmoid_fast(tt)) : uint16_t(0);
      } else if (inj && tg == 0 && qm < M) {
        inj[size_t(qm) * HC + (r - rank)] = f32_to_bf16(sigmoid_fast(tt) * 2.0f);
      }
    }
  }
  zero_block(lds, steps, 1024);
  __syncthreads();
  // 2. stage lo (8 rows x rank) in operand order with its group sums
  {
    const int units = rank / 8;
    const int i = threadIdx.x;  // 8 * units <= 512 <= 1024 threads, a multiple of 64
    if (i < 8 * units) {        // uniform per wave
      const int m = i & 7, u = i >> 3;
      const uint4 val = *reinterpret_cast<const uint4*>(lo + m * rank + u * 8);
      stage_unit(lds, steps, val, m, u);
    }
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
  if (threadIdx.x >= 128 || mm >= M || tg * 16 + cj >= hidden) return;
  float sum = 0.0f;
#pragma unroll
  for (int s = 0; s < HC; ++s) {
    const float inv = __builtin_amdgcn_rsqf(fmaf_(ssq[s * 8 + mm], inv_hidden, eps));
    const float x = round_bf16((bf16_to_f32(hv[s]) * inv) * (bf16_to_f32(wv[s]) + 1.0f));
    const float p = round_bf16(yt[mm * 64 + s * 16 + cj]);
    sum = sum + round_bf16(sigmoid_fast(p) * x);
  }
  mixed[size_t(mm) * hidden + c] = f32_to_bf16(round_bf16(sum) * 0.25f);
}

int down_waves(int hidden) {
  const int sps = hidden / sk::kSuper;
  return sps < kMaxDownWaves ? sps : kMaxDownWaves;
}

}  // namespace

int hc_fused_npad(int n_down) { return ((n_down + 63) / 64) * 64; }
size_t hc_fused_part_bytes(int n_down) {
  return (size_t(4) * 8 * hc_fused_npad(n_down) + 4 * 8) * sizeof(float);
}

bool hc_fused_supported(const QWeight& down, const QWeight& up, int hc, int hidden, int rank) {
  if (hc != 4 || hidden % sk::kSuper != 0 || hidden > 2048) return false;
  const int sps = hidden / sk::kSuper;
  const int spw = sps / down_waves(hidden);
  return sps % down_waves(hidden) == 0 && (spw == 1 || spw == 2) && down.k == hc * hidden &&
         down.group_size == 64 && up.group_size == 64 && down.bits == up.bits && up.k == rank &&
         up.n == hc * hidden && rank % 256 == 0 && rank <= 512 &&
         (down.n == rank || down.n == rank + hc) &&
         hc_fused_npad(down.n) * 2 <= 1024 &&
         (down.bits == 4 || down.bits == 5 || down.bits == 6 || down.bits == 8);
}

int hc_fused(const QWeight& down, const QWeight& up, const uint16_t* h, const uint16_t* scale,
             int M, int hc, int hidden, int rank, float eps, float* part, uint16_t* mixed,
             uint16_t* inj, hipStream_t s) {
  if (M < 1 || M > 8 || !hc_fused_supported(down, up, hc, hidden, rank)) return MX_EUNSUPPORTED;
  const int npad = hc_fused_npad(down.n);
  float* ssq = part + size_t(4) * 8 * npad;
  const int waves = down_waves(hidden);
  const int spw = (hidden / sk::kSuper) / waves;
  const dim3 g1((down.n + 15) / 16, hc);
  const int lb2 = sk::stage_bytes(rank / sk::kSuper);
  switch (down.bits * 4 + spw) {
#define MX_HC(B, W)                                                                           \
  case B * 4 + W:                                                                             \
    hipLaunchKernelGGL((hc_down_kernel<B, W>), g1, dim3(64 * waves), 0, s, down, h, scale, M, \
                       hidden, part, ssq, npad);                                              \
    break;
    MX_HC(4, 1) MX_HC(4, 2) MX_HC(5, 1) MX_HC(5, 2) MX_HC(6, 1) MX_HC(6, 2) MX_HC(8, 1)
    MX_HC(8, 2)
#undef MX_HC
    default: return MX_EUNSUPPORTED;
  }
  const dim3 g2((hidden + 15) / 16);
  switch (down.bits * 8 + rank / sk::kSuper) {
#define MX_UP(B, S)                                                                           \
  case B * 8 + S:                                                                             \
    hipLaunchKernelGGL((hc_up_kernel<B, S>), g2, dim3(1024), lb2, s, up, part, ssq, npad,       \
                       down.n, rank, M, hidden, eps, h, scale, mixed, inj);                   \
    break;
    MX_UP(4, 2) MX_UP(4, 4) MX_UP(5, 2) MX_UP(5, 4) MX_UP(6, 2) MX_UP(6, 4) MX_UP(8, 2)
    MX_UP(8, 4)
#undef MX_UP
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
