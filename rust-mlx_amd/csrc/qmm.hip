// Fast affine-quantised projections on the gfx950 matrix cores (MFMA), for
// 1..kQmmMaxRows activation rows (blocks of 16 rows): decode batches, verify
// blocks and prefill chunks.
//
// Replaces the same reference interfaces as the exact kernels (qmv_kernel /
// gather_qmm of Linear::forward_rows, src/weights.rs:111-202; the expert
// gate/up/down of MoE::parts, src/hybrid.rs:192-287) with the arithmetic of
// qmm_core.hpp: results agree with the exact kernels to fp32 summation-order
// differences (a bf16 ulp or so after rounding), not bit for bit.
//
// A workgroup has four waves.  K is split across SK waves (each takes a
// contiguous range of 64-value groups); their fp32 partials are added in wave
// order in LDS before the epilogue, so the result is deterministic.
#include "common.hpp"
#include "kernels.hpp"
#include "qmm_core.hpp"

namespace mx {

namespace {

constexpr int kMaxGroups = 128;  // K <= 8192

__device__ __forceinline__ float sigmoid_bf16(float x) {
  const float e = round_bf16(expf_(__builtin_fabsf(x)));
  const float d = round_bf16(1.0f + e);
  const float y = round_bf16(1.0f / d);
  return x < 0.0f ? y : round_bf16(1.0f - y);
}

__host__ __device__ inline int split_k(int k) {
  const int G = k >> 6;
  return G >= 16 ? 4 : G >= 8 ? 2 : 1;
}

// Adds the SK partials of each tile group in wave order; returns true on the
// waves that hold the sums (k-part 0).
template <int NT, int SK>
__device__ __forceinline__ bool reduce_split(floatx4_t (&y)[NT], float* red) {
  if constexpr (SK == 1) {
    return true;
  } else {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kp = wave % SK;
    if (kp != 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        *reinterpret_cast<floatx4_t*>(red + ((wave * NT + t) * 64 + lane) * 4) = y[t];
    }
    __syncthreads();
    if (kp != 0) return false;
#pragma unroll
    for (int p = 1; p < SK; ++p)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const floatx4_t v = *reinterpret_cast<const floatx4_t*>(red + (((wave + p) * NT + t) * 64 + lane) * 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) y[t][r] = y[t][r] + v[r];
      }
    return true;
  }
}

// ---------------------------------------------------------------------------
// Dense projections with the proj.hip epilogues.  NT = 1 for kPlain, kHcDown
// and kHcWrite (tile group = 16 rows); NT = 4 for kHcUpMix (the four streams
// s*H + c of 16 columns c).
// blockIdx.y: the block of 16 activation rows (rows 16 blockIdx.y .. +15).
template <int BITS, int NT, int SK>
__global__ __launch_bounds__(256) void dense_kernel(QWeight w, const uint16_t* __restrict__ x,
                                                    int64_t x_stride, int M, ProjEpilogue e) {
  __shared__ float red[(SK > 1 ? 4 * NT * 64 * 4 : 4)];
  const int m0 = 16 * blockIdx.y;
  x += size_t(m0) * x_stride;
  M = min(M - m0, 16);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, kq = lane >> 4;
  const int tg = blockIdx.x * (4 / SK) + wave / SK;
  const int kp = wave % SK;
  const int n = w.n;
  int base, wrow[NT];
  bool live;
  if constexpr (NT == 4) {  // kHcUpMix
    base = tg * 16;
    live = base < e.hidden;
#pragma unroll
    for (int t = 0; t < 4; ++t) wrow[t] = min(t * e.hidden + base + j, n - 1);
  } else {
    base = tg * 16 * NT;
    live = base < n;
#pragma unroll
    for (int t = 0; t < NT; ++t) wrow[t] = min(base + 16 * t + j, n - 1);
  }
  floatx4_t y[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) y[t] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int G = w.k >> 6;
  if (live) {
    TileRow tr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) tr[t] = tile_row(w.codes, w.scales, w.biases, w.k, BITS, wrow[t]);
    qmm_tiles<BITS, NT>(tr, j < M ? x + size_t(j) * x_stride : nullptr, G * kp / SK,
                        G * (kp + 1) / SK, y);
  }
  if (!reduce_split<NT, SK>(y, red) || !live) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (4 * kq + r >= M) continue;
    const int m = m0 + 4 * kq + r;
    if constexpr (NT == 4) {
      const int c = base + j;
      if (c >= e.hidden) continue;
      float sum = 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float p = round_bf16(y[s][r]);
        const float xn = bf16_to_f32(e.xn[size_t(m) * e.xn_stride + size_t(s) * e.hidden + c]);
        sum = sum + round_bf16(sigmoid_bf16(p) * xn);
      }
      e.y[size_t(m) * e.y_stride + c] = f32_to_bf16(round_bf16(sum) / 4.0f);
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int row = base + 16 * t + j;
        if (row >= n) continue;
        const float v = y[t][r];
        if (e.mode == kPlain) {
          e.y[size_t(m) * e.y_stride + row] = f32_to_bf16(v);
        } else if (e.mode == kHcDown) {
          const float tt = round_bf16(round_bf16(v) / float(e.hc));
          if (row < e.rank)
            e.y[size_t(m) * e.y_stride + row] = f32_to_bf16(tt * sigmoid_bf16(tt));
          else
            e.aux[size_t(m) * e.aux_stride + (row - e.rank)] = f32_to_bf16(sigmoid_bf16(tt) * 2.0f);
        } else {  // kHcWrite
          const float vb = round_bf16(v);
          for (int s = 0; s < e.hc; ++s) {
            uint16_t* res = e.y + size_t(m) * e.y_stride + size_t(s) * n + row;
            const float inj = round_bf16(vb * bf16_to_f32(e.aux[size_t(m) * e.aux_stride + s]));
            *res = f32_to_bf16(bf16_to_f32(*res) + inj);
          }
        }
      }
    }
  }
}

template <int BITS, int NT, int SK>
void launch_dense(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
                  hipStream_t s) {
  const int tiles = NT == 4 ? (e.hidden + 15) / 16 : (w.n + 16 * NT - 1) / (16 * NT);
  const int per_block = 4 / SK;
  const int blocks = (tiles + per_block - 1) / per_block;
  hipLaunchKernelGGL((dense_kernel<BITS, NT, SK>), dim3(blocks, (m + 15) / 16), dim3(256), 0, s, w,
                     x, xs, m, e);
}

template <int BITS, int NT>
void dense_sk(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
              hipStream_t s) {
  switch (split_k(w.k)) {
    case 4: launch_dense<BITS, NT, 4>(w, x, xs, m, e, s); break;
    case 2: launch_dense<BITS, NT, 2>(w, x, xs, m, e, s); break;
    default: launch_dense<BITS, NT, 1>(w, x, xs, m, e, s); break;
  }
}

template <int BITS>
void dense_bits(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
                hipStream_t s) {
  if (e.mode == kHcUpMix)
    dense_sk<BITS, 4>(w, x, xs, m, e, s);
  else
    dense_sk<BITS, 1>(w, x, xs, m, e, s);
}

// ---------------------------------------------------------------------------
// Prefill GEMM (more than 16 activation rows): a workgroup computes a tile of
// 64 weight rows x 128 activation rows over the groups [g0, g1) of its k
// slice (blockIdx.z); wave (wn, wm) of its 2 x 2 waves owns 32 weight rows
// (two 16-row tiles) x 64 activation rows (four 16-row tiles).  The
// activations of two groups (128 k) at a time are staged in LDS once for the
// four waves (eight lanes per 128-byte row piece), and so are the weights of
// those groups, dequantised (gemm_dq_kernel); the next two groups'
// activations are in flight while the matrix cores work on these, and the
// weights of the stage after are requested too.  With a k split the
// workgroups write fp32 partials and gemm_reduce_kernel adds them in slice
// order before the epilogue.
constexpr int kGemmM = 128;          // activation rows per workgroup
constexpr int kGemmN = 64;           // weight rows per workgroup
constexpr int kGemmLd = 64 + 8;      // padded LDS row (bf16) of one group
constexpr int kGemmStage = 2;        // groups staged per barrier pair

// The projection epilogues of one output (activation row m, weight row `row`).
__device__ __forceinline__ void gemm_epilogue(const ProjEpilogue& e, int n, int m, int row,
                                              float v) {
  if (e.mode == kPlain) {
    e.y[size_t(m) * e.y_stride + row] = f32_to_bf16(v);
  } else if (e.mode == kHcDown) {
    const float tt = round_bf16(round_bf16(v) / float(e.hc));
    if (row < e.rank)
      e.y[size_t(m) * e.y_stride + row] = f32_to_bf16(tt * sigmoid_bf16(tt));
    else
      e.aux[size_t(m) * e.aux_stride + (row - e.rank)] = f32_to_bf16(sigmoid_bf16(tt) * 2.0f);
  } else {  // kHcWrite
    const float vb = round_bf16(v);
    for (int s = 0; s < e.hc; ++s) {
      uint16_t* res = e.y + size_t(m) * e.y_stride + size_t(s) * n + row;
      const float inj = round_bf16(vb * bf16_to_f32(e.aux[size_t(m) * e.aux_stride + s]));
      *res = f32_to_bf16(bf16_to_f32(*res) + inj);
    }
  }
}

// Prefill projections: the weights dequantised once per workgroup.  Each
// stage, thread t turns 32 codes of weight row t / 4 (k piece t % 4 of the
// stage's 128; BITS 32-bit words) into w = s q + b in fp32 and stores two bf16 parts in LDS,
// hi = bf16(w) and lo = bf16(w - hi) (w - hi is exact in fp32; hi + lo is w
// to within 2^-17 |w|).  The waves then multiply plain tiles, x hi + x lo
// into fp32 accumulators over the whole slice, with no per-group scale work
// per output (the exact-code form applies s and b to every output of every
// group, and its 128 q offset cancels in fp32).  Lane quarter kq of MFMA step
// st covers k = 16 kq + 8 st .. + 7 of a group on both operands.
constexpr int kDqLd = 2 * 64 + 8;  // padded LDS row (bf16) of a stage's weights
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__host__ __device__ constexpr int gemm_dq_lds() {
  return (kGemmStage * kGemmM * kGemmLd + 2 * kGemmN * kDqLd) * 2;
}

// Code v (0..31) of a 32-code piece held in BITS words, value v at bit BITS v.
template <int BITS, int V>
__device__ __forceinline__ uint32_t piece_code(const uint32_t (&w)[BITS]) {
  constexpr int bit = BITS * V, word = bit >> 5, off = bit & 31;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if constexpr (off + BITS <= 32)
    return (w[word] >> off) & mask;
  else
    return __builtin_amdgcn_alignbit(w[word + 1], w[word], uint32_t(off)) & mask;
}

// MIX (kHcUpMix, no k split): the workgroup's 64 weight rows are the four
// streams' rows s H + c of 16 columns c (blockIdx.x 16 .. + 15), and the
// epilogue mixes the four streams of each column through LDS with
// dense_kernel's kHcUpMix arithmetic.
template <int BITS, bool SPLIT, bool MIX = false>
__global__ __launch_bounds__(256) void gemm_dq_kernel(QWeight w, const uint16_t* __restrict__ x,
                                                      int64_t x_stride, int M, int per,
                                                      ProjEpilogue e) {
  extern __shared__ __align__(16) uint16_t dq_lds[];
  auto xs = reinterpret_cast<uint16_t (*)[kGemmM][kGemmLd]>(dq_lds);
  auto wh = reinterpret_cast<uint16_t (*)[kDqLd]>(dq_lds + kGemmStage * kGemmM * kGemmLd);
  auto wl = wh + kGemmN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, kq = lane >> 4;
  const int wn = wave & 1, wm = wave >> 1;
  const int n = w.n, G = w.k >> 6;
  const int mb = blockIdx.y * kGemmM;
  const int gbeg = blockIdx.z * per;
  const int gend = min(G, gbeg + per);
  // dequantising role: weight row dr of the workgroup, 32-value piece dp
  const int dr = tid >> 2, dp = tid & 3;
  const int cb = int(blockIdx.x) * 16;  // MIX: the workgroup's first column
  const int wrow = MIX ? (dr >> 4) * e.hidden + min(cb + (dr & 15), e.hidden - 1)
                       : min(int(blockIdx.x) * kGemmN + dr, n - 1);
  const uint32_t* crow = w.codes + size_t(wrow) * (size_t(w.k) * BITS / 32);
  const uint16_t* srow = w.scales + size_t(wrow) * G;
  const uint16_t* brow = w.biases + size_t(wrow) * G;
  const int sc8 = tid & 7, sr0 = tid >> 3;
  uint4 xv[8];
  auto load_x = [&](int g0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = sr0 + 32 * (i & 3), g = g0 + (i >> 2);
      if (mb + r < M && g < gend)
        xv[i] = *reinterpret_cast<const uint4*>(x + size_t(mb + r) * x_stride + 64 * g + 8 * sc8);
      else
        xv[i] = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  struct StageW {
    uint32_t c[BITS];  // 32 codes of row dr, group g0 + dp / 2, half dp % 2
    uint16_t sc, bi;
  };
  auto load_w = [&](int g0, StageW& st) {
    const int g = min(g0 + (dp >> 1), gend - 1);
    const uint32_t* src = crow + 2 * BITS * g + BITS * (dp & 1);
    if constexpr (BITS % 4 == 0) {  // 16-byte aligned pieces
#pragma unroll
      for (int i = 0; i < BITS / 4; ++i) {
        const uint4 v = reinterpret_cast<const uint4*>(src)[i];
        st.c[4 * i] = v.x;
        st.c[4 * i + 1] = v.y;
        st.c[4 * i + 2] = v.z;
        st.c[4 * i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < BITS; ++i) st.c[i] = src[i];
    }
    st.sc = srow[g];
    st.bi = brow[g];
  };
  floatx4_t y[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) y[t][u] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
  StageW w0, w1;
  load_w(gbeg, w0);
  load_w(gbeg + kGemmStage, w1);
  load_x(gbeg);
  for (int g0 = gbeg; g0 < gend; g0 += kGemmStage) {
    StageW w2;
    load_w(g0 + 2 * kGemmStage, w2);  // two stages ahead (clamped to the slice)
    __syncthreads();                  // every wave is done with the previous stage's LDS
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = sr0 + 32 * (i & 3), gs = i >> 2;
      *reinterpret_cast<uint4*>(&xs[gs][r][8 * sc8]) = xv[i];
    }
    {
      const float sc = bf16_to_f32(w0.sc), bi = bf16_to_f32(w0.bi);
      uint32_t qv[32];
      [&]<int... V>(std::integer_sequence<int, V...>) {
        ((qv[V] = piece_code<BITS, V>(w0.c)), ...);
      }(std::make_integer_sequence<int, 32>{});
#pragma unroll
      for (int q8 = 0; q8 < 4; ++q8) {  // codes 8 q8 .. + 7
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v0 = fmaf_(sc, float(qv[8 * q8 + 2 * i]), bi);
          const float v1 = fmaf_(sc, float(qv[8 * q8 + 2 * i + 1]), bi);
          const bf16x2_t h = {__bf16(v0), __bf16(v1)};
          const uint32_t hb = __builtin_bit_cast(uint32_t, h);
          const bf16x2_t l = {__bf16(v0 - u2f(hb << 16)), __bf16(v1 - u2f(hb & 0xffff0000u))};
          hw[i] = hb;
          lw[i] = __builtin_bit_cast(uint32_t, l);
        }
        const int col = 32 * dp + 8 * q8;
        *reinterpret_cast<uint4*>(&wh[dr][col]) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *reinterpret_cast<uint4*>(&wl[dr][col]) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
      }
    }
    __syncthreads();
    if (g0 + kGemmStage < gend) load_x(g0 + kGemmStage);  // next stage, in flight
#pragma unroll
    for (int s = 0; s < kGemmStage; ++s) {
      if (g0 + s >= gend) break;  // uniform
      uint4 bh[2][2], bl[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int nr = wn * 32 + 16 * t + j, col = 64 * s + 16 * kq + 8 * st;
          bh[t][st] = *reinterpret_cast<const uint4*>(&wh[nr][col]);
          bl[t][st] = *reinterpret_cast<const uint4*>(&wl[nr][col]);
        }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int row = wm * 64 + 16 * u + j;
        const uint4* xp = reinterpret_cast<const uint4*>(&xs[s][row][16 * kq]);
        const uint4 a0 = xp[0], a1 = xp[1];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          y[t][u] = mfma_bf16(a0, bh[t][0], y[t][u]);
          y[t][u] = mfma_bf16(a1, bh[t][1], y[t][u]);
          y[t][u] = mfma_bf16(a0, bl[t][0], y[t][u]);
          y[t][u] = mfma_bf16(a1, bl[t][1], y[t][u]);
        }
      }
    }
    w0 = w1;
    w1 = w2;
  }
  if constexpr (MIX) {
    // stream s = 2 wn + t of column cb + j: bf16(p) into LDS [row][s][column]
    __syncthreads();  // the last stage's operands are read
    float* ex = reinterpret_cast<float*>(dq_lds);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ex[((wm * 64 + 16 * u + 4 * kq + r) * 4 + 2 * wn + t) * 16 + j] = round_bf16(y[t][u][r]);
    __syncthreads();
    for (int i = tid; i < kGemmM * 16; i += 256) {
      const int ml = i >> 4, c = i & 15, m = mb + ml;
      if (m >= M || cb + c >= e.hidden) continue;
      float sum = 0.0f;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const float xn =
            bf16_to_f32(e.xn[size_t(m) * e.xn_stride + size_t(st) * e.hidden + cb + c]);
        sum = sum + round_bf16(sigmoid_bf16(ex[(ml * 4 + st) * 16 + c]) * xn);
      }
      e.y[size_t(m) * e.y_stride + cb + c] = f32_to_bf16(round_bf16(sum) / 4.0f);
    }
    return;
  }
  const int nb = blockIdx.x * kGemmN + wn * 32;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = nb + 16 * t + j;
    if (row >= n) continue;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mb + wm * 64 + 16 * u + 4 * kq + r;
        if (m >= M) continue;
        if constexpr (SPLIT)
          e.part[(size_t(blockIdx.z) * M + m) * n + row] = y[t][u][r];
        else
          gemm_epilogue(e, n, m, row, y[t][u][r]);
      }
  }
}

// The k slices' partial sums added in slice order, then the epilogue.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(int n, int M, int slices,
                                                          ProjEpilogue e) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= size_t(M) * n) return;
  const int m = int(i / n), row = int(i - size_t(m) * n);
  float v = e.part[i];
  for (int z = 1; z < slices; ++z) v = v + e.part[size_t(z) * M * n + i];
  gemm_epilogue(e, n, m, row, v);
}

template <int BITS>
void launch_gemm(const QWeight& w, const uint16_t* x, int64_t xs, int m, const ProjEpilogue& e,
                 hipStream_t s) {
  const int G = w.k >> 6;
  const int mb = (m + kGemmM - 1) / kGemmM;
  if (e.mode == kHcUpMix) {  // four streams of 16 columns per workgroup, no k split
    const void* fn = reinterpret_cast<const void*>(gemm_dq_kernel<BITS, false, true>);
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, gemm_dq_lds()) !=
        hipSuccess)
      return;
    hipLaunchKernelGGL((gemm_dq_kernel<BITS, false, true>), dim3((e.hidden + 15) / 16, mb, 1),
                       dim3(256), gemm_dq_lds(), s, w, x, xs, m, G, e);
    return;
  }
  const int nb = (w.n + kGemmN - 1) / kGemmN;
  // split k across workgroups until the grid has about 256 workgroups, each
  // slice at least four groups, when the workspace holds the partials
  int slices = 1;
  while (nb * mb * slices < 256 && G / (2 * slices) >= 4 && e.part &&
         size_t(2 * slices) * m * w.n <= e.part_floats)
    slices *= 2;
  const int per = (G + slices - 1) / slices;
  const dim3 grid(nb, mb, slices);
  // the LDS above the default 64 KiB needs the kernel attribute
  const void* fn = slices == 1 ? reinterpret_cast<const void*>(gemm_dq_kernel<BITS, false>)
                               : reinterpret_cast<const void*>(gemm_dq_kernel<BITS, true>);
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, gemm_dq_lds()) !=
      hipSuccess)
    return;
  if (slices == 1)
    hipLaunchKernelGGL((gemm_dq_kernel<BITS, false>), grid, dim3(256), gemm_dq_lds(), s, w, x,
                       xs, m, per, e);
  else
    hipLaunchKernelGGL((gemm_dq_kernel<BITS, true>), grid, dim3(256), gemm_dq_lds(), s, w, x,
                       xs, m, per, e);
  if (slices > 1) {
    const size_t outs = size_t(m) * w.n;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3(unsigned((outs + 255) / 256)), dim3(256), 0, s,
                       w.n, m, slices, e);
  }
}

// ---------------------------------------------------------------------------
// Experts.  One workgroup serves one plan entry (an expert and the rows that
// chose it) for 4/SK tile groups.  gate/up: NT = 2 (the gate tile and the up
// tile of the same 16 rows), SwiGLU in the epilogue.  down: NT = 1, the route
// score product in the epilogue.
__device__ __forceinline__ QWeight expert_weight(const QBank& b, int expert, const QWeight& shared) {
  if (expert < 0) return shared;
  const size_t cs = size_t(b.n) * b.k * b.bits / 32;
  const size_t ss = size_t(b.n) * (b.k / b.group_size);
  return QWeight{b.codes + cs * expert, b.scales + ss * expert, b.biases + ss * expert, b.n, b.k,
                 b.bits, b.group_size};
}

template <int BITS, int SK>
__global__ __launch_bounds__(256) void expert_gate_up_kernel(const uint16_t* __restrict__ x,
                                                             const MoePlan* __restrict__ plan,
                                                             int top_k, QBank gate, QBank up,
                                                             QWeight sgate, QWeight sup,
                                                             uint16_t* __restrict__ h, int hs) {
  __shared__ float red[(SK > 1 ? 4 * 2 * 64 * 4 : 4)];
  const int entry = blockIdx.y;
  if (entry >= plan->count) return;
  const int M = plan->m[entry];
  const int expert = plan->expert[entry];
  const QWeight gw = expert_weight(gate, expert, sgate);
  const QWeight uw = expert_weight(up, expert, sup);
  const int hidden = gate.k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, kq = lane >> 4;
  int row_of[8], slot_of[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    row_of[i] = plan->row[entry][i];
    slot_of[i] = plan->slot[entry][i];
  }
  const int tg = blockIdx.x * (4 / SK) + wave / SK;
  const int kp = wave % SK;
  const int inter = gw.n;
  const int base = tg * 16;
  const bool live = base < inter;
  floatx4_t y[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  const int G = hidden >> 6;
  if (live) {
    const int row = min(base + j, inter - 1);
    const TileRow tr[2] = {tile_row(gw.codes, gw.scales, gw.biases, hidden, BITS, row),
                           tile_row(uw.codes, uw.scales, uw.biases, hidden, BITS, row)};
    const uint16_t* xa = j < M ? x + size_t(row_of[j & 7]) * hidden : nullptr;
    qmm_tiles<BITS, 2>(tr, xa, G * kp / SK, G * (kp + 1) / SK, y);
  }
  if (!reduce_split<2, SK>(y, red) || !live) return;
  const int c = base + j;
  if (c >= inter) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * kq + r;
    if (m >= M) continue;
    const float gv = round_bf16(y[0][r]);
    const float uv = round_bf16(y[1][r]);
    const float silu = round_bf16(gv * sigmoid_bf16(gv));
    h[(size_t(row_of[m]) * (top_k + 1) + slot_of[m]) * hs + c] = f32_to_bf16(silu * uv);
  }
}

template <int BITS, int SK>
__global__ __launch_bounds__(256) void expert_down_kernel(const uint16_t* __restrict__ h,
                                                          const MoePlan* __restrict__ plan,
                                                          const uint16_t* __restrict__ scores,
                                                          int top_k, QBank down, QWeight sdown,
                                                          uint16_t* __restrict__ p, int hs) {
  __shared__ float red[(SK > 1 ? 4 * 64 * 4 : 4)];
  const int entry = blockIdx.y;
  if (entry >= plan->count) return;
  const int M = plan->m[entry];
  const int expert = plan->expert[entry];
  const QWeight dw = expert_weight(down, expert, sdown);
  const int hidden = dw.n, inter = dw.k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, kq = lane >> 4;
  int row_of[8], slot_of[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    row_of[i] = plan->row[entry][i];
    slot_of[i] = plan->slot[entry][i];
  }
  const int tg = blockIdx.x * (4 / SK) + wave / SK;
  const int kp = wave % SK;
  const int base = tg * 16;
  const bool live = base < hidden;
  floatx4_t y[1] = {{0.0f, 0.0f, 0.0f, 0.0f}};
  const int G = inter >> 6;
  if (live) {
    const TileRow tr[1] = {tile_row(dw.codes, dw.scales, dw.biases, inter, BITS,
                                    min(base + j, hidden - 1))};
    const uint16_t* xa =
        j < M ? h + (size_t(row_of[j & 7]) * (top_k + 1) + slot_of[j & 7]) * hs : nullptr;
    qmm_tiles<BITS, 1>(tr, xa, G * kp / SK, G * (kp + 1) / SK, y);
  }
  if (!reduce_split<1, SK>(y, red) || !live) return;
  const int c = base + j;
  if (c >= hidden) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * kq + r;
    if (m >= M) continue;
    const bool routed = slot_of[m] < top_k;
    const float dv = round_bf16(y[0][r]);
    const float sc = routed ? bf16_to_f32(scores[size_t(row_of[m]) * top_k + slot_of[m]]) : 1.0f;
    p[(size_t(row_of[m]) * (top_k + 1) + slot_of[m]) * hidden + c] = f32_to_bf16(routed ? dv * sc : dv);
  }
}

// ---------------------------------------------------------------------------
// Experts of a prefill chunk over a ChunkPlan: one workgroup serves one item
// (an expert and up to 16 of its routes) for a range of output rows, each
// wave over the whole depth (qmm_tiles, the arithmetic of expert_gate_up_kernel
// / expert_down_kernel without the split of k).  Lane j (of each quarter)
// holds member j's row and slot; the epilogue's rows 4 kq .. +3 read theirs
// from those lanes.
struct ChunkItem {
  int m, expert;
  int row, slot;      // this lane's member (j < m; else member m - 1)
  int erow[4], eslot[4];  // members 4 kq .. 4 kq + 3 (epilogue rows)
};

__device__ __forceinline__ ChunkItem chunk_item(const ChunkPlan* __restrict__ plan, int item) {
  ChunkItem it;
  it.m = plan->m[item];
  it.expert = plan->expert[item];
  const int start = plan->start[item];
  const int lane = threadIdx.x & 63;
  const int j = lane & 15, kq = lane >> 4;
  const int mj = j < it.m ? j : it.m - 1;
  it.row = plan->row[start + mj];
  it.slot = plan->slot[start + mj];
#pragma unroll
  for (int r = 0; r < 4; ++r) {  // every lane takes part in the shuffles
    it.erow[r] = __shfl(it.row, 4 * kq + r, 64);
    it.eslot[r] = __shfl(it.slot, 4 * kq + r, 64);
  }
  return it;
}

// gate/up: wave w of the workgroup takes 32 rows of the gate and the same 32
// rows of the up matrix (four tiles sharing the activation operands and their
// group sums) over the whole depth, so a workgroup streams 128 rows of each
// matrix and the item's plan is read once per 256 KB of 4-bit weights.
// SX: the item's rows pass through LDS once per batch of four groups for the
// four waves (qmm_tiles_sx) instead of every wave reading them; every wave
// then takes part in the batches' barriers, past the matrix's rows too.
template <int BITS, bool SX>
__global__ __launch_bounds__(256) void chunk_gate_up_kernel(const uint16_t* __restrict__ x,
                                                            const ChunkPlan* __restrict__ plan,
                                                            int top_k, QBank gate, QBank up,
                                                            QWeight sgate, QWeight sup,
                                                            uint16_t* __restrict__ h, int hs) {
  if (int(blockIdx.y) >= plan->nitems) return;
  const ChunkItem it = chunk_item(plan, blockIdx.y);
  const QWeight gw = expert_weight(gate, it.expert, sgate);
  const QWeight uw = expert_weight(up, it.expert, sup);
  const int hidden = gate.k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, kq = lane >> 4;
  const int inter = gw.n;
  const int base = (blockIdx.x * 4 + wave) * 32;
  if (!SX && base >= inter) return;
  const int r0 = min(base + j, inter - 1), r1 = min(base + 16 + j, inter - 1);
  const TileRow tr[4] = {tile_row(gw.codes, gw.scales, gw.biases, hidden, BITS, r0),
                         tile_row(gw.codes, gw.scales, gw.biases, hidden, BITS, r1),
                         tile_row(uw.codes, uw.scales, uw.biases, hidden, BITS, r0),
                         tile_row(uw.codes, uw.scales, uw.biases, hidden, BITS, r1)};
  floatx4_t y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (SX) {
    __shared__ __align__(16) uint16_t xs[16 * kSxLd];
    const int sr = threadIdx.x >> 4;  // the member this thread stages (lane sr holds its row)
    const int srow = __shfl(it.row, sr, 64);
    qmm_tiles_sx<BITS, 4, 256>(tr, sr < it.m ? x + size_t(srow) * hidden : nullptr, xs,
                               j < it.m ? j : -1, 0, hidden >> 6, y);
    if (base >= inter) return;
  } else {
    const uint16_t* xa = j < it.m ? x + size_t(it.row) * hidden : nullptr;
    qmm_tiles<BITS, 4>(tr, xa, 0, hidden >> 6, y);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int c = base + 16 * t + j;
    if (c >= inter) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (4 * kq + r >= it.m) continue;
      const float gv = round_bf16(y[t][r]);
      const float uv = round_bf16(y[2 + t][r]);
      const float silu = round_bf16(gv * sigmoid_bf16(gv));
      h[(size_t(it.erow[r]) * (top_k + 1) + it.eslot[r]) * hs + c] = f32_to_bf16(silu * uv);
    }
  }
}

// The gate/up on 32-row tiles (qmm_tiles32_sx): wave w takes gate and
// up rows base .. base + 31, lane l the row base + l % 32 of both; lane l
// holds activation rows 8 (i / 4) + 4 (l / 32) + i % 4 (i < 8) of its column.
template <int BITS>
__global__ __launch_bounds__(256) void chunk_gate_up32_kernel(const uint16_t* __restrict__ x,
                                                              const ChunkPlan* __restrict__ plan,
                                                              int top_k, QBank gate, QBank up,
                                                              QWeight sgate, QWeight sup,
                                                              uint16_t* __restrict__ h, int hs) {
  if (int(blockIdx.y) >= plan->nitems) return;
  const ChunkItem it = chunk_item(plan, blockIdx.y);
  const QWeight gw = expert_weight(gate, it.expert, sgate);
  const QWeight uw = expert_weight(up, it.expert, sup);
  const int hidden = gate.k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, hf = lane >> 5;
  const int inter = gw.n;
  const int base = (blockIdx.x * 4 + wave) * 32;
  const int r0 = min(base + j, inter - 1);
  const TileRow tr[2] = {tile_row(gw.codes, gw.scales, gw.biases, hidden, BITS, r0),
                         tile_row(uw.codes, uw.scales, uw.biases, hidden, BITS, r0)};
  // the members of this lane's activation rows (lane m % 16 holds member m)
  int er[8], es[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ar = 8 * (i >> 2) + 4 * hf + (i & 3);
    er[i] = __shfl(it.row, ar, 64);
    es[i] = __shfl(it.slot, ar, 64);
  }
  floatx16_t y[2] = {{}, {}};
  __shared__ __align__(16) uint16_t xs[16 * kSxLd];
  const int sr = threadIdx.x >> 4;  // the member this thread stages (lane sr holds its row)
  const int srow = __shfl(it.row, sr, 64);
  qmm_tiles32_sx<BITS, 2, 256>(tr, sr < it.m ? x + size_t(srow) * hidden : nullptr, xs,
                         (lane & 31) < it.m ? (lane & 31) : -1, 0, hidden >> 6, y);
  const int c = base + j;
  if (c >= inter) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ar = 8 * (i >> 2) + 4 * hf + (i & 3);
    if (ar >= it.m) continue;
    const float gv = round_bf16(y[0][i]);
    const float uv = round_bf16(y[1][i]);
    const float silu = round_bf16(gv * sigmoid_bf16(gv));
    h[(size_t(er[i]) * (top_k + 1) + es[i]) * hs + c] = f32_to_bf16(silu * uv);
  }
}

// The down on 32-row tiles (qmm_tiles32_sx): wave w takes rows base .. base +
// 63 as two tiles, lane l rows base + 32 t + l % 32.
template <int BITS>
__global__ __launch_bounds__(256) void chunk_down32_kernel(const uint16_t* __restrict__ h,
                                                           const ChunkPlan* __restrict__ plan,
                                                           const uint16_t* __restrict__ scores,
                                                           int top_k, QBank down, QWeight sdown,
                                                           uint16_t* __restrict__ p, int hs) {
  if (int(blockIdx.y) >= plan->nitems) return;
  const ChunkItem it = chunk_item(plan, blockIdx.y);
  const QWeight dw = expert_weight(down, it.expert, sdown);
  const int hidden = dw.n, inter = dw.k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, hf = lane >> 5;
  const int base = (blockIdx.x * 4 + wave) * 64;
  TileRow tr[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
    tr[t] = tile_row(dw.codes, dw.scales, dw.biases, inter, BITS, min(base + 32 * t + j, hidden - 1));
  int er[8], es[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ar = 8 * (i >> 2) + 4 * hf + (i & 3);
    er[i] = __shfl(it.row, ar, 64);
    es[i] = __shfl(it.slot, ar, 64);
  }
  floatx16_t y[2] = {{}, {}};
  __shared__ __align__(16) uint16_t xs[16 * kSxLd];
  const int sr = threadIdx.x >> 4;  // the member this thread stages (lane sr holds it)
  const int srow = __shfl(it.row, sr, 64), sslot = __shfl(it.slot, sr, 64);
  qmm_tiles32_sx<BITS, 2, 256>(
      tr, sr < it.m ? h + (size_t(srow) * (top_k + 1) + sslot) * hs : nullptr, xs,
      j < it.m ? j : -1, 0, inter >> 6, y);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ar = 8 * (i >> 2) + 4 * hf + (i & 3);
    if (ar >= it.m) continue;
    const bool routed = es[i] < top_k;
    const float sc = routed ? bf16_to_f32(scores[size_t(er[i]) * top_k + es[i]]) : 1.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c = base + 32 * t + j;
      if (c >= hidden) continue;
      const float dv = round_bf16(y[t][i]);
      p[(size_t(er[i]) * (top_k + 1) + es[i]) * hidden + c] = f32_to_bf16(routed ? dv * sc : dv);
    }
  }
}

// down: wave w takes 64 rows (four tiles) over the whole depth; a workgroup
// streams 256 rows of the expert's down matrix.
template <int BITS, bool SX>
__global__ __launch_bounds__(256) void chunk_down_kernel(const uint16_t* __restrict__ h,
                                                         const ChunkPlan* __restrict__ plan,
                                                         const uint16_t* __restrict__ scores,
                                                         int top_k, QBank down, QWeight sdown,
                                                         uint16_t* __restrict__ p, int hs) {
  if (int(blockIdx.y) >= plan->nitems) return;
  const ChunkItem it = chunk_item(plan, blockIdx.y);
  const QWeight dw = expert_weight(down, it.expert, sdown);
  const int hidden = dw.n, inter = dw.k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, kq = lane >> 4;
  const int base = (blockIdx.x * 4 + wave) * 64;
  if (!SX && base >= hidden) return;
  TileRow tr[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    tr[t] = tile_row(dw.codes, dw.scales, dw.biases, inter, BITS, min(base + 16 * t + j, hidden - 1));
  floatx4_t y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (SX) {
    __shared__ __align__(16) uint16_t xs[16 * kSxLd];
    const int sr = threadIdx.x >> 4;  // the member this thread stages (lane sr holds it)
    const int srow = __shfl(it.row, sr, 64), sslot = __shfl(it.slot, sr, 64);
    qmm_tiles_sx<BITS, 4, 256>(
        tr, sr < it.m ? h + (size_t(srow) * (top_k + 1) + sslot) * hs : nullptr, xs,
        j < it.m ? j : -1, 0, inter >> 6, y);
    if (base >= hidden) return;
  } else {
    const uint16_t* xa = j < it.m ? h + (size_t(it.row) * (top_k + 1) + it.slot) * hs : nullptr;
    qmm_tiles<BITS, 4>(tr, xa, 0, inter >> 6, y);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (4 * kq + r >= it.m) continue;
    const int row = it.erow[r], slot = it.eslot[r];
    const bool routed = slot < top_k;
    const float sc = routed ? bf16_to_f32(scores[size_t(row) * top_k + slot]) : 1.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int c = base + 16 * t + j;
      if (c >= hidden) continue;
      const float dv = round_bf16(y[t][r]);
      p[(size_t(row) * (top_k + 1) + slot) * hidden + c] = f32_to_bf16(routed ? dv * sc : dv);
    }
  }
}

}  // namespace

bool qmm_supported(const QWeight& w) {
  return w.group_size == 64 && w.k % 64 == 0 && (w.k >> 6) <= kMaxGroups &&
         (w.bits == 4 || w.bits == 5 || w.bits == 6 || w.bits == 8);
}

int qmm(const QWeight& w, const uint16_t* x, int64_t x_stride, int m, const ProjEpilogue& e,
        hipStream_t s) {
  if (!qmm_supported(w) || m < 1 || m > kQmmMaxRows) return MX_EUNSUPPORTED;
  if (e.mode == kHcUpMix && e.hidden * 4 != w.n) return MX_EUNSUPPORTED;
  if (e.mode == kConv) return MX_EUNSUPPORTED;
  if (m > 16) {  // prefill rows: the staged GEMM
    switch (w.bits) {
      case 4: launch_gemm<4>(w, x, x_stride, m, e, s); break;
      case 5: launch_gemm<5>(w, x, x_stride, m, e, s); break;
      case 6: launch_gemm<6>(w, x, x_stride, m, e, s); break;
      default: launch_gemm<8>(w, x, x_stride, m, e, s); break;
    }
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
  }
  switch (w.bits) {
    case 4: dense_bits<4>(w, x, x_stride, m, e, s); break;
    case 5: dense_bits<5>(w, x, x_stride, m, e, s); break;
    case 6: dense_bits<6>(w, x, x_stride, m, e, s); break;
    default: dense_bits<8>(w, x, x_stride, m, e, s); break;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int qmm_gate_up(const uint16_t* x, const MoePlan* plan, int rows, int top_k, const QBank& gate,
                const QBank& up, const QWeight& sgate, const QWeight& sup, uint16_t* h,
                hipStream_t s) {
  const int routes = rows * top_k + 1;
  const int hs = gate.n > sgate.n ? gate.n : sgate.n;
  const int SK = split_k(gate.k);
  const int tiles = (hs + 15) / 16;
  const dim3 grid((tiles + 4 / SK - 1) / (4 / SK), routes);
#define MX_GU(B, K)                                                                          \
  if (gate.bits == B && SK == K) {                                                           \
    hipLaunchKernelGGL((expert_gate_up_kernel<B, K>), grid, dim3(256), 0, s, x, plan, top_k, \
                       gate, up, sgate, sup, h, hs);                                         \
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;                               \
  }
  MX_GU(4, 4) MX_GU(4, 2) MX_GU(4, 1) MX_GU(5, 4) MX_GU(5, 2) MX_GU(5, 1)
  MX_GU(6, 4) MX_GU(6, 2) MX_GU(6, 1) MX_GU(8, 4) MX_GU(8, 2) MX_GU(8, 1)
#undef MX_GU
  return MX_EUNSUPPORTED;
}

int qmm_down(const uint16_t* h, const MoePlan* plan, const uint16_t* scores, int rows, int top_k,
             int inter, int shared_inter, const QBank& down, const QWeight& sdown, uint16_t* p,
             hipStream_t s) {
  const int routes = rows * top_k + 1;
  const int hs = inter > shared_inter ? inter : shared_inter;
  // one split for both depths: the shallower one's waves cover fewer groups
  const int kmin = down.k < sdown.k ? down.k : sdown.k;
  const int SK = split_k(kmin);
  const int tiles = (down.n + 15) / 16;
  const dim3 grid((tiles + 4 / SK - 1) / (4 / SK), routes);
#define MX_DN(B, K)                                                                         \
  if (down.bits == B && SK == K) {                                                          \
    hipLaunchKernelGGL((expert_down_kernel<B, K>), grid, dim3(256), 0, s, h, plan, scores,  \
                       top_k, down, sdown, p, hs);                                          \
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;                              \
  }
  MX_DN(4, 4) MX_DN(4, 2) MX_DN(4, 1) MX_DN(5, 4) MX_DN(5, 2) MX_DN(5, 1)
  MX_DN(6, 4) MX_DN(6, 2) MX_DN(6, 1) MX_DN(8, 4) MX_DN(8, 2) MX_DN(8, 1)
#undef MX_DN
  return MX_EUNSUPPORTED;
}

// The 32-row tile forms (4- and 8-bit codes, whole batches of four groups).
bool chunk_w32_ok(int bits, int k) { return (bits == 4 || bits == 8) && (k >> 6) % 4 == 0; }

int qmm_chunk_gate_up(const uint16_t* x, const ChunkPlan* plan, int rows, int experts, int top_k,
                      const QBank& gate, const QBank& up, const QWeight& sgate,
                      const QWeight& sup, uint16_t* h, hipStream_t s) {
  const int hs = gate.n > sgate.n ? gate.n : sgate.n;
  const dim3 grid((hs + 127) / 128, chunk_max_items(rows, experts, top_k));
  const bool sx = (gate.k >> 6) % 4 == 0;  // whole batches of four groups
  if (sx && gate.bits == sgate.bits && chunk_w32_ok(gate.bits, gate.k) &&
      chunk_w32_ok(sgate.bits, sgate.k)) {
    // 32-row tiles: each lane reads a group's 32 codes with 16-byte loads
    if (gate.bits == 4)
      hipLaunchKernelGGL((chunk_gate_up32_kernel<4>), grid, dim3(256), 0, s, x, plan, top_k,
                         gate, up, sgate, sup, h, hs);
    else
      hipLaunchKernelGGL((chunk_gate_up32_kernel<8>), grid, dim3(256), 0, s, x, plan, top_k,
                         gate, up, sgate, sup, h, hs);
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
  }
  switch (gate.bits) {
#define MX_GU(B)                                                                              \
  case B:                                                                                     \
    if (sx)                                                                                   \
      hipLaunchKernelGGL((chunk_gate_up_kernel<B, true>), grid, dim3(256), 0, s, x, plan,     \
                         top_k, gate, up, sgate, sup, h, hs);                                 \
    else                                                                                      \
      hipLaunchKernelGGL((chunk_gate_up_kernel<B, false>), grid, dim3(256), 0, s, x, plan,    \
                         top_k, gate, up, sgate, sup, h, hs);                                 \
    break;
    MX_GU(4) MX_GU(5) MX_GU(6) MX_GU(8)
#undef MX_GU
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int qmm_chunk_down(const uint16_t* h, const ChunkPlan* plan, const uint16_t* scores, int rows,
                   int experts, int top_k, int inter, int shared_inter, const QBank& down,
                   const QWeight& sdown, uint16_t* p, hipStream_t s) {
  const int hs = inter > shared_inter ? inter : shared_inter;
  const dim3 grid((down.n + 255) / 256, chunk_max_items(rows, experts, top_k));
  const bool sx = (down.k >> 6) % 4 == 0 && (sdown.k >> 6) % 4 == 0;
  if (sx && down.bits == sdown.bits && chunk_w32_ok(down.bits, down.k) &&
      chunk_w32_ok(sdown.bits, sdown.k)) {
    if (down.bits == 4)
      hipLaunchKernelGGL((chunk_down32_kernel<4>), grid, dim3(256), 0, s, h, plan, scores, top_k,
                         down, sdown, p, hs);
    else
      hipLaunchKernelGGL((chunk_down32_kernel<8>), grid, dim3(256), 0, s, h, plan, scores, top_k,
                         down, sdown, p, hs);
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
  }
  switch (down.bits) {
#define MX_DN(B)                                                                              \
  case B:                                                                                     \
    if (sx)                                                                                   \
      hipLaunchKernelGGL((chunk_down_kernel<B, true>), grid, dim3(256), 0, s, h, plan, scores, \
                         top_k, down, sdown, p, hs);                                          \
    else                                                                                      \
      hipLaunchKernelGGL((chunk_down_kernel<B, false>), grid, dim3(256), 0, s, h, plan,       \
                         scores, top_k, down, sdown, p, hs);                                  \
    break;
    MX_DN(4) MX_DN(5) MX_DN(6) MX_DN(8)
#undef MX_DN
    default: return MX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
