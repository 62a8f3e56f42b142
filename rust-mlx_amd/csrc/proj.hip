// Quantised projections with fused epilogues, the hyper-connection grouped
// norm and the embedding gather (gfx950).
//
// Every projection shares qmv_core's fixed order (bit-identical to mx_qmv);
// only what happens to the fp32 row sums differs:
//   kPlain   y = bf16(v)                                       Linear::forward
//   kHcDown  rows < rank: lo = activate(bf16(v)) = silu(v/hc)  compiled::activate
//            rows >= rank: inj = 2*sigmoid(bf16(v)/hc)         compiled::injection
//   kHcUpMix rows {c, c+H, .., c+(hc-1)H}: mixed[c] = mean_s sigmoid(p_s) * xn_s
//                                                              compiled::mix
//   kHcWrite residual[s][c] = bf16(residual + bf16(bf16(v) * inj[s]))
//                                                              HyperConnection::write
// (reference src/hybrid.rs:78-105, src/compiled.rs:46-86).  Element-wise
// steps follow MLX's bf16 graphs with one bf16 rounding per operation.
#include "common.hpp"
#include "kernels.hpp"
#include "xq_core.hpp"
#include "qmv_core.hpp"

namespace mx {

namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ float sigmoid_bf16(float x) {
  const float e = round_bf16(expf_(__builtin_fabsf(x)));
  const float d = round_bf16(1.0f + e);
  const float y = round_bf16(1.0f / d);
  return x < 0.0f ? y : round_bf16(1.0f - y);
}

template <int BITS, int M>
__global__ __launch_bounds__(256) void proj_kernel(QWeight w, const uint16_t* __restrict__ x,
                                                   int64_t x_stride, int L, ProjEpilogue e) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & (L - 1);
  const int lg = lane / L;
  const int group = (blockIdx.x * kWaves + wave) * (64 / L) + lg;
  const int n = w.n;
  int rows[kQRows];
  int row0;
  if (e.mode == kHcUpMix) {
    // lane group c computes rows c + s*H (kQRows == hc streams)
    row0 = group;
    if (row0 >= e.hidden) return;
#pragma unroll
    for (int r = 0; r < kQRows; ++r) rows[r] = row0 + r * e.hidden;
  } else {
    row0 = group * kQRows;
    if (row0 >= n) return;
#pragma unroll
    for (int r = 0; r < kQRows; ++r) rows[r] = min(row0 + r, n - 1);
  }
  const uint16_t* xrow[M];
#pragma unroll
  for (int m = 0; m < M; ++m) xrow[m] = x + size_t(m) * x_stride;
  float out[M][kQRows];
  qmv_core<BITS, M>(w.codes, w.scales, w.biases, w.k, w.group_size, xrow, rows, li, L, out);
  if (li != 0) return;
  switch (e.mode) {
    case kPlain:
#pragma unroll
      for (int r = 0; r < kQRows; ++r)
        if (row0 + r < n)
#pragma unroll
          for (int m = 0; m < M; ++m) e.y[size_t(m) * e.y_stride + row0 + r] = f32_to_bf16(out[m][r]);
      break;
    case kHcDown: {
      const float hcf = float(e.hc);
#pragma unroll
      for (int r = 0; r < kQRows; ++r) {
        const int row = row0 + r;
        if (row >= n) continue;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float t = round_bf16(round_bf16(out[m][r]) / hcf);
          if (row < e.rank) {
            e.y[size_t(m) * e.y_stride + row] = f32_to_bf16(t * sigmoid_bf16(t));
          } else {
            e.aux[size_t(m) * e.aux_stride + (row - e.rank)] = f32_to_bf16(sigmoid_bf16(t) * 2.0f);
          }
        }
      }
      break;
    }
    case kHcUpMix: {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float sum = 0.0f;
#pragma unroll
        for (int s = 0; s < kQRows; ++s) {
          const float p = round_bf16(out[m][s]);
          const float xn = bf16_to_f32(e.xn[size_t(m) * e.xn_stride + size_t(s) * e.hidden + row0]);
          sum = sum + round_bf16(sigmoid_bf16(p) * xn);
        }
        e.y[size_t(m) * e.y_stride + row0] = f32_to_bf16(round_bf16(sum) / float(kQRows));
      }
      break;
    }
    case kHcWrite: {
#pragma unroll
      for (int r = 0; r < kQRows; ++r) {
        const int c = row0 + r;
        if (c >= n) continue;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float v = round_bf16(out[m][r]);
          for (int s = 0; s < e.hc; ++s) {
            uint16_t* res = e.y + size_t(m) * e.y_stride + size_t(s) * n + c;
            const float inj = round_bf16(v * bf16_to_f32(e.aux[size_t(m) * e.aux_stride + s]));
            *res = f32_to_bf16(bf16_to_f32(*res) + inj);
          }
        }
      }
      break;
    }
  }
}

template <int BITS, int M>
void launch_proj(const QWeight& w, const uint16_t* x, int64_t xs, const ProjEpilogue& e,
                 hipStream_t s) {
  const int L = qmv_lanes_per_row(w.k);
  const int groups_per_block = kWaves * (64 / L);
  const int groups = e.mode == kHcUpMix ? e.hidden : (w.n + kQRows - 1) / kQRows;
  const int blocks = (groups + groups_per_block - 1) / groups_per_block;
  hipLaunchKernelGGL((proj_kernel<BITS, M>), dim3(blocks), dim3(64 * kWaves), 0, s, w, x, xs, L, e);
}

template <int BITS>
void proj_m(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
            hipStream_t s) {
  switch (m) {
    case 1: launch_proj<BITS, 1>(w, x, xs, e, s); break;
    case 2: launch_proj<BITS, 2>(w, x, xs, e, s); break;
    case 3: launch_proj<BITS, 3>(w, x, xs, e, s); break;
    case 4: launch_proj<BITS, 4>(w, x, xs, e, s); break;
    case 5: launch_proj<BITS, 5>(w, x, xs, e, s); break;
    case 6: launch_proj<BITS, 6>(w, x, xs, e, s); break;
    case 7: launch_proj<BITS, 7>(w, x, xs, e, s); break;
    default: launch_proj<BITS, 8>(w, x, xs, e, s); break;
  }
}

// ---------------------------------------------------------------------------
// Grouped zero-centred RMS norm of the hc streams (compiled::norm over
// [hc, H], src/compiled.rs:22-28; grouped_norm src/hybrid.rs:39-44):
//   y = bf16((x * rsqrt(mean(x^2) + eps)) * (scale + 1))   in f32.
// One workgroup (256 threads) per (row, stream); thread t sums x^2 over
// columns t, t+256, ... in order; xor butterfly per wave; waves summed in order.
// plane (nullable, rows <= 8): also writes the exact-integer operand plane of
// y (xq_core.hpp), the hc * hidden values of row blockIdx.y as one K-long row
template <int K>
__global__ __launch_bounds__(256) void hc_norm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ scale,
                                                      int hidden, float eps,
                                                      uint16_t* __restrict__ y,
                                                      char* __restrict__ plane) {
  // K > 0: hidden == 256 K, every value loaded once into registers (thread t
  // holds columns t, t + 256, ...); K == 0: any hidden, loops over columns
  __shared__ float red[4];
  extern __shared__ __align__(16) uint16_t ys[];  // the normalised stream (plane only)
  const int s = blockIdx.x;
  const int row = blockIdx.y;
  const int hc = gridDim.x;
  const int t = threadIdx.x;
  const uint16_t* xr = x + (size_t(row) * hc + s) * hidden;
  const uint16_t* sc = scale + size_t(s) * hidden;
  uint16_t* yr = y + (size_t(row) * hc + s) * hidden;
  float xv[K > 0 ? K : 1], sv[K > 0 ? K : 1];
  float acc = 0.0f;
  if constexpr (K > 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      xv[k] = bf16_to_f32(xr[t + 256 * k]);
      sv[k] = bf16_to_f32(sc[t + 256 * k]);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) acc = acc + xv[k] * xv[k];
  } else {
    for (int c = t; c < hidden; c += 256) {
      const float v = bf16_to_f32(xr[c]);
      acc = acc + v * v;
    }
  }
  for (int o = 32; o > 0; o >>= 1) acc = acc + __shfl_xor(acc, o, 64);
  if ((t & 63) == 0) red[t >> 6] = acc;
  __syncthreads();
  const float total = ((red[0] + red[1]) + red[2]) + red[3];
  const float inv = 1.0f / __builtin_sqrtf(total / float(hidden) + eps);
  if constexpr (K > 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const uint16_t o = f32_to_bf16((xv[k] * inv) * (sv[k] + 1.0f));
      yr[t + 256 * k] = o;
      if (plane) ys[t + 256 * k] = o;
    }
  } else {
    for (int c = t; c < hidden; c += 256) {
      const uint16_t o = f32_to_bf16((bf16_to_f32(xr[c]) * inv) * (bf16_to_f32(sc[c]) + 1.0f));
      yr[c] = o;
      if (plane) ys[c] = o;
    }
  }
  if (!plane) return;
  __syncthreads();
  // lane l of wave w takes values 16 (l / 16) .. +15 of group w * 16 + l % 16
  // (and of every 64th group after it) and writes their operands
  const int lane = t & 63, wave = t >> 6, kb = lane >> 4;
  const int ng = hidden / xq::kGroup;
  for (int g0 = wave * 16; g0 < ng; g0 += 64) {
    const int gl = g0 + (lane & 15);
    const bool live = gl < ng;
    float f[16];
    if (live) {
      const uint4 a = *reinterpret_cast<const uint4*>(ys + gl * xq::kGroup + 16 * kb);
      const uint4 b = *reinterpret_cast<const uint4*>(ys + gl * xq::kGroup + 16 * kb + 8);
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
    xq::digitize_unit(f, row, s * ng + gl, kb, live, plane, hc * ng);
  }
}

// Embedding rows dequantised and broadcast to hc streams
// (HybridModel::forward_hidden, src/hybrid.rs:605-612).
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* __restrict__ codes,
                                                    const uint16_t* __restrict__ scales,
                                                    const uint16_t* __restrict__ biases,
                                                    const uint32_t* __restrict__ ids, int k,
                                                    int bits, int gs, int n, int hc,
                                                    uint16_t* __restrict__ out) {
  const int i = blockIdx.y;
  const uint32_t row = min(ids[i], uint32_t(n - 1));
  const int words_per_row = (k * bits) >> 5;
  const uint32_t* rw = codes + size_t(row) * words_per_row;
  const uint32_t mask = (1u << bits) - 1u;
  for (int col = blockIdx.x * blockDim.x + threadIdx.x; col < k; col += gridDim.x * blockDim.x) {
    const int bit = col * bits;
    const int word = bit >> 5, off = bit & 31;
    uint32_t v = rw[word] >> off;
    if (off + bits > 32) v |= rw[word + 1] << (32 - off);
    const int g = col / gs;
    const float sc = bf16_to_f32(scales[size_t(row) * (k / gs) + g]);
    const float bi = bf16_to_f32(biases[size_t(row) * (k / gs) + g]);
    const uint16_t e = f32_to_bf16(sc * float(v & mask) + bi);
    for (int s = 0; s < hc; ++s) out[(size_t(i) * hc + s) * k + col] = e;
  }
}

// The MTP layer's input: the embedding projection added to every stream's
// hidden projection in bf16 (src/mtp.rs:103-106).
__global__ __launch_bounds__(256) void mtp_combine_kernel(const uint16_t* __restrict__ e,
                                                          const uint16_t* __restrict__ f,
                                                          int hc, int hidden,
                                                          uint16_t* __restrict__ y) {
  const int r = blockIdx.y;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < hc * hidden; i += gridDim.x * 256) {
    const int c = i % hidden;
    y[size_t(r) * hc * hidden + i] = f32_to_bf16(bf16_to_f32(e[size_t(r) * hidden + c]) +
                                                 bf16_to_f32(f[size_t(r) * hc * hidden + i]));
  }
}

}  // namespace

int mtp_combine(const uint16_t* e, const uint16_t* f, int rows, int hc, int hidden, uint16_t* y,
                hipStream_t s) {
  const int bx = (hc * hidden + 255) / 256;
  hipLaunchKernelGGL(mtp_combine_kernel, dim3(bx, rows), dim3(256), 0, s, e, f, hc, hidden, y);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int proj(const QWeight& w, const uint16_t* x, int64_t x_stride, int m, const ProjEpilogue& e,
         hipStream_t s) {
  if (e.mode == kHcUpMix && (e.hidden * kQRows != w.n)) return MX_EUNSUPPORTED;
  if (e.mode == kConv) return MX_EUNSUPPORTED;
  switch (w.bits) {
    case 4: proj_m<4>(w, x, x_stride, m, e, s); break;
    case 5: proj_m<5>(w, x, x_stride, m, e, s); break;
    case 6: proj_m<6>(w, x, x_stride, m, e, s); break;
    case 8: proj_m<8>(w, x, x_stride, m, e, s); break;
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int hc_norm(const uint16_t* x, const uint16_t* scale, int rows, int hc, int hidden, float eps,
            uint16_t* y, hipStream_t s, char* plane) {
  if (plane && (rows > 8 || hidden % xq::kGroup != 0)) return MX_EUNSUPPORTED;
  const int lb = plane ? hidden * 2 : 0;
  if (hidden == 2048)
    hipLaunchKernelGGL(hc_norm_kernel<8>, dim3(hc, rows), dim3(256), lb, s, x, scale, hidden, eps,
                       y, plane);
  else if (hidden == 4096)
    hipLaunchKernelGGL(hc_norm_kernel<16>, dim3(hc, rows), dim3(256), lb, s, x, scale, hidden,
                       eps, y, plane);
  else if (hidden % 256 == 0 && hidden <= 1024)
    hipLaunchKernelGGL(hidden == 256 ? hc_norm_kernel<1>
                                     : hidden == 512 ? hc_norm_kernel<2>
                                                     : hidden == 768 ? hc_norm_kernel<3>
                                                                     : hc_norm_kernel<4>,
                       dim3(hc, rows), dim3(256), lb, s, x, scale, hidden, eps, y, plane);
  else
    hipLaunchKernelGGL(hc_norm_kernel<0>, dim3(hc, rows), dim3(256), lb, s, x, scale, hidden, eps,
                       y, plane);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int embed(const QWeight& w, const uint32_t* ids, int count, int hc, uint16_t* out,
          hipStream_t s) {
  const int bx = (w.k + 255) / 256;
  hipLaunchKernelGGL(embed_kernel, dim3(bx, count), dim3(256), 0, s, w.codes, w.scales, w.biases,
                     ids, w.k, w.bits, w.group_size, w.n, hc, out);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
